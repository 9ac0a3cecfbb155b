"""GPU parity: HIP kernels (through the C ABI / the Torch front end) against
the CPU oracle on the same seeded inputs.

Tolerances (stated per the north star):
  integer / index outputs: bit-exact;
  fp32 outputs and gradients: max|gpu - oracle| <= 1e-5 * max|oracle| per tensor
  (oracle in fp64).
"""

import ctypes

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import tiga as tg
from tiga import _native
from tiga.graph import build_row_plan, build_transpose
from oracle import ref

from graphs import skewed_csr

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
RTOL32 = 1e-5


def rel_err(actual, expected):
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    scale = np.abs(e).max() if e.size else 0.0
    if scale == 0:
        return float(np.abs(a).max()) if a.size else 0.0
    return float(np.abs(a - e).max() / scale)


def to_dev(a, dtype):
    return torch.as_tensor(np.asarray(a), device=DEV).to(dtype)


@pytest.fixture(autouse=True)
def _strict():
    tg.config.strict = True
    yield
    tg.config.strict = False


# ---- graph indexing --------------------------------------------------------

@pytest.mark.parametrize("idx", [torch.int32, torch.int64])
@pytest.mark.parametrize("case", [
    dict(seed=0, n_dst=200, n_src=150, mean_deg=5),
    dict(seed=1, n_dst=70000, n_src=90001, mean_deg=6, hubs=(3000, 700), hot_src=5,
         hot_frac=0.02),
    dict(seed=2, n_dst=5, n_src=3, mean_deg=0, empty_frac=1.0),
])
def test_transpose_bit_exact(idx, case):
    print(f"transpose {case} {idx}", flush=True)
    rp, col = skewed_csr(**case)
    n_dst, n_src = case["n_dst"], case["n_src"]
    rpt, colt, perm, inv = build_transpose(to_dev(rp, idx), to_dev(col, idx), n_dst, n_src)
    e_rpt, e_colt, e_perm = ref.transpose(rp, col, n_src)
    assert rpt.cpu().numpy().tolist() == e_rpt.tolist()
    assert colt.cpu().numpy().tolist() == e_colt.tolist()
    assert perm.cpu().numpy().tolist() == e_perm.tolist()
    e_inv = np.empty_like(e_perm)
    e_inv[e_perm] = np.arange(e_perm.size)
    assert inv.cpu().numpy().tolist() == e_inv.tolist()
    # determinism: a second run is bit-identical
    rpt2, colt2, perm2, inv2 = build_transpose(to_dev(rp, idx), to_dev(col, idx), n_dst, n_src)
    assert torch.equal(colt, colt2) and torch.equal(perm, perm2) and torch.equal(inv, inv2)


@pytest.mark.parametrize("idx", [torch.int32, torch.int64])
def test_destination_index_bit_exact(idx):
    rp, col = skewed_csr(3, 5000, 5000, hubs=(900,))
    out = torch.empty(col.size, dtype=torch.int64, device=DEV)
    _native.call("tgx_destination_index", to_dev(rp, idx).data_ptr(), 64 if idx == torch.int64 else 32,
                 rp.size - 1, col.size, out.data_ptr(), 64, _native.stream_of(out))
    assert out.cpu().numpy().tolist() == ref.destination_index(rp).tolist()


@pytest.mark.parametrize("idx", [torch.int32, torch.int64])
@pytest.mark.parametrize("n_dst", [1, 4096, 100003])
def test_row_plan_bit_exact(idx, n_dst):
    print(f"row plan n_dst={n_dst} {idx}", flush=True)
    rp, _ = skewed_csr(4, n_dst, 1000, mean_deg=20, hubs=(5000, 513, 512, 1025)[:n_dst],
                       empty_frac=0.3)
    for wave_max, chunk in ((512, 512), (16, 64)):
        h = build_row_plan(to_dev(rp, idx), n_dst, wave_max=wave_max, chunk_edges=chunk)
        rows, n_empty, n_wave, n_split, chunk_off = ref.row_plan(rp, wave_max, chunk)
        p = h.plan
        assert (p.n_empty, p.n_wave, p.n_split) == (n_empty, n_wave, n_split)
        assert h.rows[:n_dst].cpu().numpy().tolist() == rows.tolist()
        assert h.chunk_offsets.cpu().numpy().tolist() == chunk_off.tolist()
        assert p.n_chunks == int(chunk_off[-1])


# ---- sum reducer -----------------------------------------------------------

class WeightedSum(tg.MessagePassing):
    reducer = tg.sum()

    def edge(self, src, dst, edge):
        return edge.weight * src.x


class PlainSum(tg.MessagePassing):
    reducer = tg.sum()

    def edge(self, src, dst, edge):
        return src.x


def test_readme_known_answer_on_gpu():
    graph = tg.Graph.from_csr(torch.tensor([0, 2, 3, 5], device=DEV),
                              torch.tensor([0, 2, 1, 0, 1], device=DEV), num_src=3)
    x = torch.tensor([1.0, 2.0, 3.0], device=DEV, requires_grad=True)
    w = torch.tensor([2.0, 3.0, 4.0, 5.0, 6.0], device=DEV, requires_grad=True)
    k = WeightedSum()
    out = k(graph=graph, src={"x": x}, dst={}, edge={"weight": w})
    dx, dw = torch.autograd.grad(out.sum(), (x, w))
    assert k.last_variant.backend == "hip"
    assert out.tolist() == [11.0, 8.0, 17.0]
    assert dx.tolist() == [7.0, 10.0, 3.0]
    assert dw.tolist() == [1.0, 3.0, 2.0, 1.0, 2.0]


@pytest.mark.parametrize("F_", [1, 3, 4, 64, 100, 300])
@pytest.mark.parametrize("idx", [torch.int32, torch.int64])
def test_sum_fwd_bwd_parity(F_, idx):
    print(f"sum F={F_} {idx}", flush=True)
    rp, col = skewed_csr(10 + F_, 3000, 2500, mean_deg=8, hubs=(1500, 600), hot_src=7,
                         hot_frac=0.3)
    rng = np.random.default_rng(F_)
    x = rng.standard_normal((2500, F_)).astype(np.float32)
    w = rng.random(col.size).astype(np.float32)
    dout = rng.standard_normal((3000, F_)).astype(np.float32)
    graph = tg.Graph.from_csr(to_dev(rp, idx), to_dev(col, idx), num_src=2500)
    xt = to_dev(x, torch.float32).requires_grad_(True)
    wt = to_dev(w, torch.float32).requires_grad_(True)
    k = WeightedSum()
    out = k(graph=graph, src={"x": xt}, dst={}, edge={"weight": wt})
    assert k.last_variant.backend == "hip"
    out.backward(to_dev(dout, torch.float32))
    e_out = ref.sum_fwd(rp, col, x, w)
    e_dx, e_dw = ref.sum_bwd(rp, col, x, w, dout)
    assert rel_err(out.detach().cpu(), e_out) <= RTOL32
    assert rel_err(xt.grad.cpu(), e_dx) <= RTOL32
    assert rel_err(wt.grad.cpu(), e_dw) <= RTOL32


# 16-bit features: the message w * x has Torch's promoted dtype, as in the
# reference's eager reduce_sum (reducer_oracle.py:44-57): bf16 x with bf16 (or
# no) weights sums to bf16, bf16 x with fp32 weights to fp32.  The kernels
# multiply and add in fp32 and round once per output.  Bars: against float64
# math, 1e-2 of the largest |value| for a 16-bit output (one rounding: 2^-8
# for bf16) and 1e-5 for an fp32 output (the 16-bit inputs are exact in
# fp32); against the reference's own arithmetic (bf16 products, index_add in
# bf16, on the CPU) 1e-2 plus that result's own distance from float64.
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("w_dtype", [None, "same", torch.float32])
@pytest.mark.parametrize("F_", [3, 64, 300])
def test_sum_16_bit_features(dtype, w_dtype, F_):
    print(f"sum 16-bit {dtype} w={w_dtype} F={F_}", flush=True)
    rp, col = skewed_csr(40 + F_, 3000, 2500, mean_deg=8, hubs=(1500, 600), hot_src=7,
                         hot_frac=0.3)
    rng = np.random.default_rng(F_)
    graph = tg.Graph.from_csr(to_dev(rp, torch.int64), to_dev(col, torch.int64), num_src=2500)
    xt = to_dev(rng.standard_normal((2500, F_)), dtype).requires_grad_(True)
    wd = None if w_dtype is None else (dtype if w_dtype == "same" else w_dtype)
    wt = None if wd is None else to_dev(rng.random(col.size), wd).requires_grad_(True)
    out_dtype = dtype if wd is None else torch.promote_types(dtype, wd)
    k = WeightedSum() if wt is not None else PlainSum()
    edge = {} if wt is None else {"weight": wt}
    out = k(graph=graph, src={"x": xt}, dst={}, edge=edge)
    assert k.last_variant.backend == "hip"
    assert out.dtype == out_dtype
    dout = to_dev(rng.standard_normal((3000, F_)), out_dtype)
    out.backward(dout)
    assert xt.grad.dtype == dtype and (wt is None or wt.grad.dtype == wd)
    f = lambda t: t.detach().double().cpu().numpy()
    w64 = None if wt is None else f(wt)
    e_out = ref.sum_fwd(rp, col, f(xt), w64)
    e_dx, e_dw = ref.sum_bwd(rp, col, f(xt), w64, f(dout))
    bar = 1e-2 if out_dtype != torch.float32 else RTOL32
    assert rel_err(f(out), e_out) <= bar
    # dx is rounded to the 16-bit input type.
    assert rel_err(f(xt.grad), e_dx) <= 1e-2
    if wt is not None:
        assert rel_err(f(wt.grad), e_dw) <= (1e-2 if wd != torch.float32 else RTOL32)
    # The reference's eager arithmetic in the message dtype, on the CPU.
    xc, dst = xt.detach().cpu(), torch.as_tensor(ref.destination_index(rp))
    msg = xc[torch.as_tensor(col)]
    if wt is not None:
        msg = wt.detach().cpu()[:, None] * msg
    ref16 = torch.zeros(3000, F_, dtype=msg.dtype).index_add_(0, dst, msg)
    own = rel_err(ref16.double().numpy(), e_out)
    err16 = rel_err(f(out), ref16.double().numpy())
    print(f"  out vs reference {msg.dtype} arithmetic {err16:.3e} (its own error {own:.3e})",
          flush=True)
    assert err16 <= 1e-2 + own


def test_sum_unweighted_and_empty_graph():
    rp, col = skewed_csr(20, 500, 400, mean_deg=3)
    x = np.random.default_rng(0).standard_normal((400, 16)).astype(np.float32)
    graph = tg.Graph.from_csr(to_dev(rp, torch.int64), to_dev(col, torch.int64), num_src=400)
    xt = to_dev(x, torch.float32).requires_grad_(True)
    out = PlainSum()(graph=graph, src={"x": xt}, dst={})
    out.sum().backward()
    assert rel_err(out.detach().cpu(), ref.sum_fwd(rp, col, x)) <= RTOL32
    assert rel_err(xt.grad.cpu(), ref.sum_bwd(rp, col, x, None, np.ones((500, 16)))[0]) <= RTOL32
    g0 = tg.Graph.from_csr(torch.zeros(4, dtype=torch.int64, device=DEV),
                           torch.zeros(0, dtype=torch.int64, device=DEV), num_src=2)
    x0 = torch.randn(2, 8, device=DEV, requires_grad=True)
    o0 = PlainSum()(graph=g0, src={"x": x0}, dst={})
    o0.sum().backward()
    assert torch.count_nonzero(o0).item() == 0 and torch.count_nonzero(x0.grad).item() == 0


@pytest.mark.parametrize("F_", [8, 3, 64])
@pytest.mark.parametrize("idx", [torch.int32, torch.int64])
def test_sum_of_edge_field_per_row(F_, idx):
    """tgx_csr_sum_fwd without a column array sums a per-edge field per
    destination row (edge ids as columns), hub rows split into chunks."""
    from tiga._ops import _reduce_rows

    print(f"edge-field row sums F={F_} {idx}", flush=True)
    rp, col = skewed_csr(31, 3000, 1000, mean_deg=9, hubs=(6000, 700))
    E = col.size
    x = np.random.default_rng(F_).standard_normal((E, F_)).astype(np.float32)
    graph = tg.Graph.from_csr(to_dev(rp, idx), to_dev(col, idx), num_src=1000)
    out = _reduce_rows(graph, to_dev(x, torch.float32))
    assert rel_err(out.cpu(), ref.sum_fwd(rp, np.arange(E), x)) <= RTOL32


# ---- GAT additive ----------------------------------------------------------

class GAT(tg.MessagePassing):
    reducer = tg.online_softmax()

    def __init__(self, a_s, a_d, slope):
        super().__init__()
        self.a_s, self.a_d, self.slope = a_s, a_d, slope

    def edge(self, src, dst, edge):
        s = F.leaky_relu((src.h * self.a_s).sum(-1) + (dst.h * self.a_d).sum(-1), self.slope)
        return self.reducer(s, src.h)


# Heads run in groups of at most 256 floats per node: (8, 64) is two groups
# of 4 heads, (3, 64) groups 2 + 1, (6, 16) 4 + 2, (5, 8) 4 + 1, (12, 32)
# 8 + 4, (2, 256) two one-head groups of 64 lanes; (1, 4) is one lane per head.
@pytest.mark.parametrize("H,D", [(8, 32), (4, 32), (2, 32), (16, 16), (4, 64), (8, 64),
                                 (3, 64), (6, 16), (5, 8), (12, 32), (1, 128), (2, 256),
                                 (1, 4)])
@pytest.mark.parametrize("idx", [torch.int32, torch.int64])
def test_gat_fwd_bwd_parity(H, D, idx):
    print(f"gat H={H} D={D} {idx}", flush=True)
    N = 2500
    rp, col = skewed_csr(100 + H, N, N, mean_deg=10, hubs=(1400, 700), hot_src=11,
                         hot_frac=0.3)
    rng = np.random.default_rng(H * D)
    h = rng.standard_normal((N, H, D)).astype(np.float32)
    a_s = (rng.standard_normal((H, D)) * 0.1).astype(np.float32)
    a_d = (rng.standard_normal((H, D)) * 0.1).astype(np.float32)
    dout = rng.standard_normal((N, H, D)).astype(np.float32)
    graph = tg.Graph.from_csr(to_dev(rp, idx), to_dev(col, idx), num_src=N)
    ht = to_dev(h, torch.float32).requires_grad_(True)
    ast = to_dev(a_s, torch.float32).requires_grad_(True)
    adt = to_dev(a_d, torch.float32).requires_grad_(True)
    k = GAT(ast, adt, 0.2)
    out = k(graph=graph, src={"h": ht}, dst={"h": ht})
    assert k.last_variant.backend == "hip"
    out.backward(to_dev(dout, torch.float32))
    e_out, _ = ref.gat_fwd(rp, col, h, a_s, a_d, 0.2)
    e_dh, e_das, e_dad = ref.gat_bwd(rp, col, h, a_s, a_d, 0.2, dout)
    assert rel_err(out.detach().cpu(), e_out) <= RTOL32
    assert rel_err(ht.grad.cpu(), e_dh) <= RTOL32
    assert rel_err(ast.grad.cpu(), e_das) <= RTOL32
    assert rel_err(adt.grad.cpu(), e_dad) <= RTOL32


class GATBipartite(tg.MessagePassing):
    reducer = tg.online_softmax()

    def __init__(self, a_s, a_d, slope):
        super().__init__()
        self.a_s, self.a_d, self.slope = a_s, a_d, slope

    def edge(self, src, dst, edge):
        s = F.leaky_relu((src.h * self.a_s).sum(-1) + (dst.g * self.a_d).sum(-1), self.slope)
        return self.reducer(s, src.h)


# Element types and bipartite relations: fp32 features at 1e-5 against
# float64, bf16 / fp16 (fp32 arithmetic, outputs rounded once) at 2e-2, with
# fp32 or same-typed attention vectors; bipartite: 1800 destinations with
# their own table g, 2600 sources with h, hub rows on both sides.
@pytest.mark.parametrize("H,D", [(8, 32), (3, 64), (2, 256), (1, 4)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("bipartite", [False, True])
@pytest.mark.parametrize("a_typed", [False, True])
def test_gat_element_types_and_bipartite_parity(H, D, dtype, bipartite, a_typed):
    print(f"gat {dtype} H={H} D={D} bipartite={bipartite} a_typed={a_typed}", flush=True)
    n_dst, n_src = (1800, 2600) if bipartite else (2500, 2500)
    rp, col = skewed_csr(200 + H, n_dst, n_src, mean_deg=10, hubs=(1400, 700), hot_src=11,
                         hot_frac=0.3)
    rng = np.random.default_rng(H * D + 1)
    mk = lambda n: to_dev(rng.standard_normal((n, H, D)), dtype)
    hs = mk(n_src)
    hd = mk(n_dst) if bipartite else hs
    dout = mk(n_dst)
    a_dtype = dtype if a_typed else torch.float32
    a_s = to_dev(rng.standard_normal((H, D)) * 0.1, a_dtype).requires_grad_(True)
    a_d = to_dev(rng.standard_normal((H, D)) * 0.1, a_dtype).requires_grad_(True)
    graph = tg.Graph.from_csr(to_dev(rp, torch.int64), to_dev(col, torch.int64), num_src=n_src)
    hst = hs.clone().requires_grad_(True)
    if bipartite:
        hdt = hd.clone().requires_grad_(True)
        k = GATBipartite(a_s, a_d, 0.2)
        out = k(graph=graph, src={"h": hst}, dst={"g": hdt})
    else:
        k = GAT(a_s, a_d, 0.2)
        out = k(graph=graph, src={"h": hst}, dst={"h": hst})
    assert k.last_variant.backend == "hip", k.explain()
    assert out.dtype == dtype
    out.backward(dout)
    f = lambda t: t.detach().double().cpu().numpy()
    e_out, _ = ref.gat_fwd(rp, col, f(hs), f(a_s), f(a_d), 0.2,
                           h_dst=f(hd) if bipartite else None)
    e_dhs, e_dhd, e_das, e_dad = ref.gat_bwd_bipartite(rp, col, f(hs), f(hd), f(a_s), f(a_d),
                                                       0.2, f(dout))
    tol = RTOL32 if dtype == torch.float32 else RTOL_BF16
    assert rel_err(f(out), e_out) <= tol
    if bipartite:
        assert hst.grad.dtype == dtype and hdt.grad.dtype == dtype
        assert rel_err(f(hst.grad), e_dhs) <= tol
        assert rel_err(f(hdt.grad), e_dhd) <= tol
    else:
        assert rel_err(f(hst.grad), e_dhs + e_dhd) <= tol
    assert a_s.grad.dtype == a_dtype
    # fp32 parameter gradients are rounded once to a 16-bit a when a is.
    a_tol = tol if a_dtype == torch.float32 else RTOL_BF16
    assert rel_err(f(a_s.grad), e_das) <= a_tol
    assert rel_err(f(a_d.grad), e_dad) <= a_tol


def test_gat_large_scores_and_determinism():
    # Scores of order 1e3 (the reference's overflow case) must stay finite.
    N, H, D = 600, 8, 32
    rp, col = skewed_csr(7, N, N, mean_deg=12, hubs=(900,))
    rng = np.random.default_rng(1)
    h = (rng.standard_normal((N, H, D)) * 30).astype(np.float32)
    a_s = rng.standard_normal((H, D)).astype(np.float32)
    a_d = rng.standard_normal((H, D)).astype(np.float32)
    graph = tg.Graph.from_csr(to_dev(rp, torch.int64), to_dev(col, torch.int64), num_src=N)
    grads = []
    for _ in range(2):
        ht = to_dev(h, torch.float32).requires_grad_(True)
        ast = to_dev(a_s, torch.float32).requires_grad_(True)
        adt = to_dev(a_d, torch.float32).requires_grad_(True)
        out = GAT(ast, adt, 0.2)(graph=graph, src={"h": ht}, dst={"h": ht})
        out.sum().backward()
        assert torch.isfinite(out).all()
        grads.append((out.detach().clone(), ht.grad.clone(), ast.grad.clone(), adt.grad.clone()))
    for a, b in zip(*grads):
        assert torch.equal(a, b)          # bit-identical reruns (no float atomics)
    e_out, _ = ref.gat_fwd(rp, col, h, a_s, a_d, 0.2)
    assert rel_err(grads[0][0].cpu(), e_out) <= RTOL32


def _gat_c_abi(graph, hs, hd, a_s, a_d, slope, dout, folded, bipartite):
    """One GAT forward + backward through the C ABI.  folded: the forward
    writes pos and the backward forms the destination terms from node rows
    (no inv_perm is passed); otherwise the per-edge destination pass."""
    from tiga._ops import _VALUE_DTYPES, _partial
    row_ptr, col = graph._kernel_csr()
    n_dst, n_src, E = graph.schema.num_dst, graph.schema.num_src, graph.num_edges
    _, H, D = hs.shape
    code, stream, bits = _VALUE_DTYPES[hs.dtype], _native.stream_of(hs), _native.idx_bits(row_ptr)
    ptr = lambda t: None if t is None else t.data_ptr()
    out = torch.empty((n_dst, H, D), dtype=hs.dtype, device=DEV)
    ns = torch.empty((n_dst, H, 4), dtype=torch.float32, device=DEV)
    pos = torch.empty((n_dst, H, D), dtype=torch.float32, device=DEV) if folded else None
    plan = graph._row_plan()
    partial = _partial(plan, 2 * H * D + 3 * H if folded else H * D + 2 * H, DEV)
    _native.call("tgx_gat_fwd", row_ptr.data_ptr(), col.data_ptr(), bits, plan.ref,
                 hs.data_ptr(), hd.data_ptr(), a_s.data_ptr(), a_d.data_ptr(), slope,
                 out.data_ptr(), ns.data_ptr(), n_dst, n_src, H, D, code, ptr(partial), ptr(pos),
                 stream)
    t = graph._transposed()
    dhs = torch.empty_like(hs)
    dhd = torch.empty_like(hd) if bipartite else dhs
    das = torch.empty((H, D), dtype=torch.float32, device=DEV)
    dad = torch.empty((H, D), dtype=torch.float32, device=DEV)
    ws_bytes = ctypes.c_size_t()
    _native.call("tgx_gat_bwd_workspace", plan.ref, t.plan.ref, E, H, D, code, int(folded),
                 ctypes.byref(ws_bytes))
    ws = torch.empty(max(ws_bytes.value, 1), dtype=torch.uint8, device=DEV)
    _native.call("tgx_gat_bwd", row_ptr.data_ptr(), col.data_ptr(), bits, plan.ref,
                 t.row_ptr_t.data_ptr(), t.col_t.data_ptr(), t.perm.data_ptr(),
                 None if folded else t.inv_perm.data_ptr(), t.plan.ref, hs.data_ptr(),
                 hd.data_ptr(), a_s.data_ptr(), a_d.data_ptr(), slope, out.data_ptr(),
                 ns.data_ptr(), ptr(pos), dout.data_ptr(), dhs.data_ptr(), dhd.data_ptr(),
                 das.data_ptr(), dad.data_ptr(), n_dst, n_src, E, H, D, code, ws.data_ptr(),
                 ws_bytes.value, stream)
    torch.cuda.synchronize()
    return out, dhs, dhd, das, dad


# The backward with the forward's pos (destination terms from node rows,
# which the Torch front end uses whenever a gradient is needed) and the
# per-edge destination pass (pos = NULL) against float64 and each other:
# hub rows split over several waves on both sides, empty rows and sources
# without out-edges, two head groups (8 x 64), 16-bit elements, and slopes
# other than 0.2 (1.0 makes the destination terms vanish).
@pytest.mark.parametrize("H,D", [(8, 32), (8, 64), (1, 4)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("bipartite", [False, True])
@pytest.mark.parametrize("slope", [0.2, -0.5, 1.0])
def test_gat_folded_and_per_edge_backwards_agree(H, D, dtype, bipartite, slope):
    print(f"gat folded H={H} D={D} {dtype} bipartite={bipartite} slope={slope}", flush=True)
    n_dst, n_src = (1800, 2600) if bipartite else (2500, 2500)
    rp, col = skewed_csr(300 + H, n_dst, n_src, mean_deg=10, hubs=(1400, 700), hot_src=11,
                         hot_frac=0.3, empty_frac=0.05)
    rng = np.random.default_rng(H * D + 7)
    mk = lambda n: to_dev(rng.standard_normal((n, H, D)), dtype)
    hs = mk(n_src)
    hd = mk(n_dst) if bipartite else hs
    dout = mk(n_dst)
    a_s = to_dev(rng.standard_normal((H, D)) * 0.1, torch.float32)
    a_d = to_dev(rng.standard_normal((H, D)) * 0.1, torch.float32)
    graph = tg.Graph.from_csr(to_dev(rp, torch.int64), to_dev(col, torch.int64), num_src=n_src)
    folded = _gat_c_abi(graph, hs, hd, a_s, a_d, slope, dout, True, bipartite)
    per_edge = _gat_c_abi(graph, hs, hd, a_s, a_d, slope, dout, False, bipartite)
    f = lambda t: t.detach().double().cpu().numpy()
    e_out, _ = ref.gat_fwd(rp, col, f(hs), f(a_s), f(a_d), slope,
                           h_dst=f(hd) if bipartite else None)
    e_dhs, e_dhd, e_das, e_dad = ref.gat_bwd_bipartite(rp, col, f(hs), f(hd), f(a_s), f(a_d),
                                                       slope, f(dout))
    expect = [e_out, e_dhs if bipartite else e_dhs + e_dhd, e_dhd, e_das, e_dad]
    tol = RTOL32 if dtype == torch.float32 else RTOL_BF16
    names = ["out", "dh_src", "dh_dst", "da_src", "da_dst"]
    for k, (name, a, b, e) in enumerate(zip(names, folded, per_edge, expect)):
        if name == "dh_dst" and not bipartite:
            continue
        if slope == 1.0 and name in ("dh_dst", "da_dst"):
            # z's gradient sums to zero over every row: the folded terms are
            # exactly zero, the per-edge ones rounding noise.
            assert not f(a).any(), name
            continue
        err_f, err_p, err_fp = rel_err(f(a), e), rel_err(f(b), e), rel_err(f(a), f(b))
        print(f"  {name}: folded {err_f:.2e}, per-edge {err_p:.2e}, between {err_fp:.2e}",
              flush=True)
        assert err_f <= tol and err_p <= tol, name
        # The two forwards are one computation; the destination terms differ
        # only in summation order.
        assert err_fp <= (1e-6 if k == 0 and dtype == torch.float32 else tol), name


# ---- dot-product attention (bf16, fp32 accumulate) ---------------------------

RTOL_BF16 = 2e-2


class DotBias(tg.MessagePassing):
    reducer = tg.online_softmax()

    def edge(self, src, dst, edge, scale):
        return self.reducer((src.k * dst.q).sum(dim=-1) * scale + edge.bias, src.v)


class DotPlain(tg.MessagePassing):
    reducer = tg.online_softmax()

    def edge(self, src, dst, edge, scale):
        return self.reducer((src.k * dst.q).sum(dim=-1) * scale, src.v)


def _bf16(a):
    return torch.as_tensor(a, device=DEV).to(torch.bfloat16)


# Heads run in groups of at most 512 values per node: (16, 64) is two groups
# of 8 heads, (3, 64) groups 2 + 1, (6, 128) 4 + 2, (5, 32) 4 + 1, (12, 16)
# 8 + 4, (1, 512) one head over 64 lanes; (1, 8) is one lane per head.
@pytest.mark.parametrize("H,D", [(4, 64), (2, 64), (8, 64), (16, 16), (16, 64), (3, 64),
                                 (6, 128), (5, 32), (12, 16), (1, 512), (1, 8)])
@pytest.mark.parametrize("idx", [torch.int32, torch.int64])
@pytest.mark.parametrize("with_bias", [True, False])
def test_dot_fwd_bwd_parity_rmat(H, D, idx, with_bias):
    from graphs import rmat_csr

    print(f"dot H={H} D={D} {idx} bias={with_bias}", flush=True)
    rp, col = rmat_csr(5, 12)                      # 4096 nodes, hubs > 512 edges
    N = rp.size - 1
    E = col.size
    rng = np.random.default_rng(H + D)
    q = _bf16(rng.standard_normal((N, H, D)))
    k = _bf16(rng.standard_normal((N, H, D)))
    v = _bf16(rng.standard_normal((N, H, D)))
    bias = to_dev(rng.standard_normal((E, H)), torch.float32)
    dout = _bf16(rng.standard_normal((N, H, D)))
    scale = 1.0 / np.sqrt(D)
    graph = tg.Graph.from_csr(to_dev(rp, idx), to_dev(col, idx), num_src=N)
    qt, kt, vt, bt = (t.clone().requires_grad_(True) for t in (q, k, v, bias))
    kernel = DotBias() if with_bias else DotPlain()
    edge = {"bias": bt} if with_bias else {}
    out = kernel(graph=graph, src={"k": kt, "v": vt}, dst={"q": qt}, edge=edge, scale=scale)
    assert kernel.last_variant.backend == "hip"
    assert out.dtype == torch.bfloat16
    out.backward(dout)
    f = lambda t: t.detach().float().cpu().numpy()
    b64 = f(bias) if with_bias else None
    e_out, _ = ref.dot_fwd(rp, col, f(q), f(k), f(v), scale, b64)
    e_dq, e_dk, e_dv, e_db = ref.dot_bwd(rp, col, f(q), f(k), f(v), scale, b64, f(dout))
    assert rel_err(f(out), e_out) <= RTOL_BF16
    assert rel_err(f(qt.grad), e_dq) <= RTOL_BF16
    assert rel_err(f(kt.grad), e_dk) <= RTOL_BF16
    assert rel_err(f(vt.grad), e_dv) <= RTOL_BF16
    if with_bias:
        assert rel_err(f(bt.grad), e_db) <= RTOL_BF16
    # empty destination rows produce exact zeros
    empty = np.flatnonzero(np.diff(rp) == 0)
    assert empty.size > 0
    assert torch.count_nonzero(out[torch.as_tensor(empty, device=DEV)]).item() == 0


def _dot_bwd_c_abi(graph, q, k, v, bias, scale, dout, stored):
    """Dot attention forward (through the front end's autograd function) and
    backward through the C ABI: stored ds (inv_perm passed: the source pass
    keeps each edge's ds for the destination pass) or recomputed."""
    from tiga._ops import _VALUE_DTYPES
    row_ptr, col = graph._kernel_csr()
    n_dst, n_src, E = graph.schema.num_dst, graph.schema.num_src, graph.num_edges
    _, H, D = q.shape
    ptr = lambda t: None if t is None else t.data_ptr()
    out = torch.empty_like(q)
    ml = torch.empty((n_dst, H, 2), dtype=torch.float32, device=DEV)
    plan, t = graph._row_plan(), graph._transposed()
    from tiga._ops import _partial
    partial = _partial(plan, H * D + 2 * H, DEV)
    code, stream, bits = _VALUE_DTYPES[q.dtype], _native.stream_of(q), _native.idx_bits(row_ptr)
    _native.call("tgx_dot_attn_fwd", row_ptr.data_ptr(), col.data_ptr(), bits, plan.ref,
                 q.data_ptr(), k.data_ptr(), v.data_ptr(), ptr(bias), scale, out.data_ptr(),
                 ml.data_ptr(), n_dst, n_src, H, D, code, ptr(partial), stream)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    dbias = None if bias is None else torch.empty((E, H), dtype=torch.float32, device=DEV)
    ws_bytes = ctypes.c_size_t()
    _native.call("tgx_dot_attn_bwd_workspace", plan.ref, t.plan.ref, E, H, D, int(stored),
                 ctypes.byref(ws_bytes))
    ws = torch.empty(max(ws_bytes.value, 1), dtype=torch.uint8, device=DEV)
    _native.call("tgx_dot_attn_bwd", row_ptr.data_ptr(), col.data_ptr(), bits, plan.ref,
                 t.row_ptr_t.data_ptr(), t.col_t.data_ptr(), t.perm.data_ptr(),
                 t.inv_perm.data_ptr() if stored else None, t.plan.ref, E, q.data_ptr(),
                 k.data_ptr(), v.data_ptr(), ptr(bias), scale, out.data_ptr(), ml.data_ptr(),
                 dout.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ptr(dbias),
                 n_dst, n_src, H, D, code, ws.data_ptr(), ws_bytes.value, stream)
    torch.cuda.synchronize()
    return dq, dk, dv, dbias


# The dot-product backward with stored ds (the front end's path) and with ds
# recomputed in the destination pass, against float64 and each other: R-MAT
# hub rows split on both sides, empty rows, two head groups (16 x 64), one
# lane per head (1 x 8), groups of more than 16 heads whose ds is stored
# without LDS staging (32 x 16, 64 x 8), with and without a bias, bf16 and
# fp32.
@pytest.mark.parametrize("H,D", [(4, 64), (16, 64), (1, 8), (32, 16), (64, 8)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("with_bias", [True, False])
def test_dot_stored_and_recomputed_ds_backwards_agree(H, D, dtype, with_bias):
    from graphs import rmat_csr

    print(f"dot stored ds H={H} D={D} {dtype} bias={with_bias}", flush=True)
    rp, col = rmat_csr(6, 12)
    N, E = rp.size - 1, col.size
    rng = np.random.default_rng(H * D + 3)
    mk = lambda: to_dev(rng.standard_normal((N, H, D)), dtype)
    q, k, v, dout = mk(), mk(), mk(), mk()
    bias = to_dev(rng.standard_normal((E, H)), torch.float32) if with_bias else None
    scale = 1.0 / np.sqrt(D)
    graph = tg.Graph.from_csr(to_dev(rp, torch.int64), to_dev(col, torch.int64), num_src=N)
    stored = _dot_bwd_c_abi(graph, q, k, v, bias, scale, dout, True)
    recomputed = _dot_bwd_c_abi(graph, q, k, v, bias, scale, dout, False)
    f = lambda t: t.detach().double().cpu().numpy()
    e = ref.dot_bwd(rp, col, f(q), f(k), f(v), scale, None if bias is None else f(bias),
                    f(dout))
    tol = RTOL32 if dtype == torch.float32 else RTOL_BF16
    for name, a, b, x in zip(("dq", "dk", "dv", "dbias"), stored, recomputed, e):
        if a is None:
            continue
        err_s, err_r, err_sr = rel_err(f(a), x), rel_err(f(b), x), rel_err(f(a), f(b))
        print(f"  {name}: stored {err_s:.2e}, recomputed {err_r:.2e}, between {err_sr:.2e}",
              flush=True)
        assert err_s <= tol and err_r <= tol, name
        # One ds formula in both paths (the source pass's dot-product order
        # differs from the destination pass's): fp32 agrees to rounding.
        if dtype == torch.float32:
            assert err_sr <= 1e-6, name


# fp32 q/k/v (fp32 arithmetic throughout: 1e-5 against float64) and fp16
# (2e-2); the bias may be any float type (read as fp32).
@pytest.mark.parametrize("H,D", [(4, 64), (3, 64), (6, 128), (1, 512), (1, 8), (16, 16)])
@pytest.mark.parametrize("idx", [torch.int32, torch.int64])
@pytest.mark.parametrize("dtype,bias_dtype", [(torch.float32, torch.float32),
                                              (torch.float16, torch.float32),
                                              (torch.float16, torch.float16),
                                              (torch.float32, None)])
def test_dot_fp32_and_fp16_parity_rmat(H, D, idx, dtype, bias_dtype):
    from graphs import rmat_csr

    print(f"dot {dtype} H={H} D={D} {idx} bias={bias_dtype}", flush=True)
    rp, col = rmat_csr(5, 12)                      # 4096 nodes, hubs > 512 edges
    N, E = rp.size - 1, col.size
    rng = np.random.default_rng(7 * H + D)
    mk = lambda: torch.as_tensor(rng.standard_normal((N, H, D)), device=DEV).to(dtype)
    q, k, v, dout = mk(), mk(), mk(), mk()
    with_bias = bias_dtype is not None
    bias = to_dev(rng.standard_normal((E, H)), bias_dtype) if with_bias else None
    scale = 1.0 / np.sqrt(D)
    graph = tg.Graph.from_csr(to_dev(rp, idx), to_dev(col, idx), num_src=N)
    qt, kt, vt = (t.clone().requires_grad_(True) for t in (q, k, v))
    bt = bias.clone().requires_grad_(True) if with_bias else None
    kernel = DotBias() if with_bias else DotPlain()
    edge = {"bias": bt} if with_bias else {}
    out = kernel(graph=graph, src={"k": kt, "v": vt}, dst={"q": qt}, edge=edge, scale=scale)
    assert kernel.last_variant.backend == "hip"
    assert out.dtype == dtype
    out.backward(dout)
    f = lambda t: t.detach().double().cpu().numpy()
    b64 = f(bias) if with_bias else None
    e_out, _ = ref.dot_fwd(rp, col, f(q), f(k), f(v), scale, b64)
    e_dq, e_dk, e_dv, e_db = ref.dot_bwd(rp, col, f(q), f(k), f(v), scale, b64, f(dout))
    tol = RTOL32 if dtype == torch.float32 else RTOL_BF16
    assert rel_err(f(out), e_out) <= tol
    assert rel_err(f(qt.grad), e_dq) <= tol
    assert rel_err(f(kt.grad), e_dk) <= tol
    assert rel_err(f(vt.grad), e_dv) <= tol
    if with_bias:
        assert bt.grad.dtype == bias_dtype
        assert rel_err(f(bt.grad), e_db) <= (tol if bias_dtype == torch.float32 else RTOL_BF16)
    empty = np.flatnonzero(np.diff(rp) == 0)
    assert torch.count_nonzero(out[torch.as_tensor(empty, device=DEV)]).item() == 0


def test_dot_hub_row_split_matches_unsplit():
    # One destination with 20000 in-edges (40 chunks) and bipartite shapes.
    rng = np.random.default_rng(3)
    n_dst, n_src, H, D = 7, 30000, 4, 64
    deg = np.array([20000, 0, 1, 511, 512, 513, 3000])
    rp = np.concatenate([[0], np.cumsum(deg)]).astype(np.int64)
    col = np.concatenate([np.sort(rng.integers(0, n_src, d)) for d in deg]).astype(np.int64)
    q = _bf16(rng.standard_normal((n_dst, H, D)))
    k = _bf16(rng.standard_normal((n_src, H, D)) * 2)
    v = _bf16(rng.standard_normal((n_src, H, D)))
    graph = tg.Graph.from_csr(to_dev(rp, torch.int64), to_dev(col, torch.int64), num_src=n_src)
    out = DotPlain()(graph=graph, src={"k": k, "v": v}, dst={"q": q}, scale=0.125)
    f = lambda t: t.detach().float().cpu().numpy()
    e_out, _ = ref.dot_fwd(rp, col, f(q), f(k), f(v), 0.125)
    assert rel_err(f(out), e_out) <= RTOL_BF16



def test_mixed_index_dtypes_and_invalid_columns_fail_closed():
    rp = np.array([0, 2, 3, 5])
    col = np.array([0, 2, 1, 0, 1])
    x = torch.tensor([1.0, 2.0, 3.0], device=DEV)
    w = torch.tensor([2.0, 3.0, 4.0, 5.0, 6.0], device=DEV)
    mixed = tg.Graph.from_csr(to_dev(rp, torch.int64), to_dev(col, torch.int32), num_src=3)
    out = WeightedSum()(graph=mixed, src={"x": x}, dst={}, edge={"weight": w})
    assert out.tolist() == [11.0, 8.0, 17.0]
    bad = tg.Graph.from_csr(to_dev(rp, torch.int64), to_dev([0, 2, 1, 0, 9], torch.int64),
                            num_src=3, validate="basic")
    with pytest.raises(ValueError, match="out-of-range"):
        WeightedSum()(graph=bad, src={"x": x}, dst={}, edge={"weight": w})

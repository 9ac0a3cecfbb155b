"""CPU twins of the device entry points (include/tgx_cpu.h), on the CPU.

The twins take the device entry points' arguments with host pointers and
walk the same row plan (whole rows, split rows chunk by chunk merged in chunk
order, empty rows).  Here they are checked against the oracle (oracle/ref.py,
pinned in tests/test_oracle.py): bit-exact for the plan, the transpose and
the destination index; 1e-5 relative for fp32 sums and GAT; 2e-2 for the
bf16/fp16 attention.  Also: results independent of the thread count, the
twins' argument and index checks, and that the device entry points reject the
same head shapes as their twins (the device shape check runs before any HIP
call, so it can be called here with zero rows).
"""

import ctypes

import numpy as np
import pytest
import torch

from tiga import _native
from oracle import ref

from graphs import rmat_csr, skewed_csr

WAVE_MAX = 512
CHUNK = 512
F32 = _native.DTYPE_F32


def call(name, *args):
    _native.call(name, *args)


def p(a):
    return None if a is None else a.ctypes.data


def rel(a, e):
    a, e = np.asarray(a, np.float64), np.asarray(e, np.float64)
    return float(np.abs(a - e).max() / max(np.abs(e).max(), 1e-300)) if e.size else 0.0


class HostPlan:
    """A tgx_row_plan over host arrays, built by the plan twins."""

    def __init__(self, rp, bits):
        n = rp.size - 1
        self.rp = np.ascontiguousarray(rp, dtype=np.int32 if bits == 32 else np.int64)
        self.rows = np.zeros(max(n, 1), np.int32)
        bounds = (ctypes.c_int64 * 3)(0, WAVE_MAX, 1 << 62)
        off = (ctypes.c_int64 * 4)()
        call("tgx_cpu_plan_degree_bins", p(self.rp), bits, n, bounds, 3, p(self.rows), off)
        self.off = list(off)
        n_split = off[3] - off[2]
        self.chunks = np.zeros(n_split + 1, np.int32)
        n_chunks = ctypes.c_int64(0)
        call("tgx_cpu_plan_split_chunks", p(self.rp), bits, p(self.rows) + 4 * off[2], n_split,
             CHUNK, p(self.chunks), ctypes.byref(n_chunks))
        self.plan = _native.RowPlan(n, off[1] - off[0], off[2] - off[1], n_split,
                                    n_chunks.value, WAVE_MAX, CHUNK, p(self.rows),
                                    p(self.chunks))

    @property
    def ref(self):
        return ctypes.byref(self.plan)


class HostGraph:
    """CSR (int32 or int64) + its transpose and both plans, all host arrays."""

    def __init__(self, rp, col, n_src, bits):
        dt = np.int32 if bits == 32 else np.int64
        self.bits, self.n_dst, self.n_src = bits, rp.size - 1, n_src
        self.rp = np.ascontiguousarray(rp, dtype=dt)
        self.col = np.ascontiguousarray(col, dtype=dt)
        self.E = int(rp[-1])
        self.rpt = np.zeros(n_src + 1, np.int32)
        self.colt = np.zeros(max(self.E, 1), np.int32)
        self.perm = np.zeros(max(self.E, 1), np.int32)
        self.inv = np.zeros(max(self.E, 1), np.int32)
        call("tgx_cpu_csr_transpose", p(self.rp), p(self.col), bits, self.n_dst, n_src, self.E,
             p(self.rpt), p(self.colt), p(self.perm), p(self.inv))
        self.plan = HostPlan(self.rp, bits)
        self.plan_t = HostPlan(self.rpt, 32)


def _graph(seed, n, bits, hubs=(1400, 700)):
    rp, col = skewed_csr(seed, n, n, mean_deg=8, hubs=hubs, hot_src=5, hot_frac=0.2)
    return rp, col, HostGraph(rp, col, n, bits)


def _bf16(x):
    return torch.as_tensor(x, dtype=torch.float32).to(torch.bfloat16)


def _raw(t16):
    return np.ascontiguousarray(t16.view(torch.int16).numpy())


def _from_raw(raw, dtype):
    return torch.from_numpy(raw.copy()).view(dtype).float().numpy()


# ---- graph construction and planning --------------------------------------------

@pytest.mark.parametrize("bits", [32, 64])
def test_plan_transpose_and_destination_index_bit_exact(bits):
    rp, col, g = _graph(1, 3000, bits)
    rows, n_empty, n_wave, n_split, chunk_off = ref.row_plan(rp, WAVE_MAX, CHUNK)
    assert g.plan.off[1] == n_empty and g.plan.off[2] - g.plan.off[1] == n_wave
    assert g.plan.off[3] - g.plan.off[2] == n_split and n_split >= 2
    assert g.plan.rows[:rp.size - 1].tolist() == rows.tolist()
    assert g.plan.chunks.tolist() == chunk_off.tolist()
    rpt, colt, perm = ref.transpose(rp, col, 3000)
    assert g.rpt.tolist() == rpt.tolist()
    assert g.colt[:g.E].tolist() == colt.tolist()
    assert g.perm[:g.E].tolist() == perm.tolist()
    assert (g.inv[g.perm[:g.E]] == np.arange(g.E)).all()
    for out_bits in (32, 64):
        out = np.zeros(g.E, np.int32 if out_bits == 32 else np.int64)
        call("tgx_cpu_destination_index", p(g.rp), bits, g.n_dst, g.E, p(out), out_bits)
        assert out.tolist() == ref.destination_index(rp).tolist()


def test_reference_bucket_bounds_through_the_twin_partition():
    # Bounds of the reference planner (lit-vector histogram scaled up).
    deg = np.repeat([8, 64, 256], [120 * 10, 7 * 10, 10])
    np.random.default_rng(2).shuffle(deg)
    rp = np.concatenate([[0], np.cumsum(deg)]).astype(np.int64)
    bounds = [8, 64, 256]
    rows = np.zeros(deg.size, np.int32)
    off = (ctypes.c_int64 * 4)()
    call("tgx_cpu_plan_degree_bins", p(rp), 64, deg.size, (ctypes.c_int64 * 3)(*bounds), 3,
         p(rows), off)
    e_rows, e_off = ref.degree_bins(rp, bounds)
    assert list(off) == e_off.tolist() and rows.tolist() == e_rows.tolist()


# ---- weighted sum --------------------------------------------------------------------

@pytest.mark.parametrize("bits", [32, 64])
@pytest.mark.parametrize("F", [1, 3, 64])
@pytest.mark.parametrize("weighted", [False, True])
def test_sum_twin_against_oracle(bits, F, weighted):
    rp, col, g = _graph(2 + F, 2500, bits)
    rng = np.random.default_rng(F)
    x = rng.standard_normal((2500, F)).astype(np.float32)
    w = rng.standard_normal(g.E).astype(np.float32) if weighted else None
    dout = rng.standard_normal((2500, F)).astype(np.float32)
    out = np.empty((2500, F), np.float32)
    call("tgx_cpu_csr_sum_fwd", p(g.rp), p(g.col), bits, g.plan.ref, p(x), p(w), p(out), 2500,
         2500, F, F32)
    assert rel(out, ref.sum_fwd(rp, col, x, w)) <= 1e-5
    dx = np.empty_like(x)
    dw = np.empty(g.E, np.float32)
    call("tgx_cpu_csr_sum_bwd", p(g.rpt), p(g.colt), p(g.perm), g.plan_t.ref, p(x), p(w),
         p(dout), p(dx), p(dw), 2500, 2500, F, F32)
    e_dx, e_dw = ref.sum_bwd(rp, col, x, w, dout)
    assert rel(dx, e_dx) <= 1e-5
    assert rel(dw, e_dw) <= 1e-5


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("F", [3, 64])
def test_sum_twin_with_16_bit_features(dtype, F):
    rp, col, g = _graph(12 + F, 2000, 32)
    rng = np.random.default_rng(F)
    x = torch.as_tensor(rng.standard_normal((2000, F)), dtype=torch.float32).to(dtype)
    dout = torch.as_tensor(rng.standard_normal((2000, F)), dtype=torch.float32).to(dtype)
    w = rng.standard_normal(g.E).astype(np.float32)
    code = _native.dtype_code(x)
    out = np.zeros((2000, F), np.int16)
    call("tgx_cpu_csr_sum_fwd", p(g.rp), p(g.col), 32, g.plan.ref, p(_raw(x)), p(w), p(out),
         2000, 2000, F, code)
    xf, gf = x.float().numpy(), dout.float().numpy()
    assert rel(_from_raw(out, dtype), ref.sum_fwd(rp, col, xf, w)) <= 1e-2
    dx = np.zeros((2000, F), np.int16)
    dw = np.empty(g.E, np.float32)
    call("tgx_cpu_csr_sum_bwd", p(g.rpt), p(g.colt), p(g.perm), g.plan_t.ref, p(_raw(x)), p(w),
         p(_raw(dout)), p(dx), p(dw), 2000, 2000, F, code)
    e_dx, e_dw = ref.sum_bwd(rp, col, xf, w, gf)
    assert rel(_from_raw(dx, dtype), e_dx) <= 1e-2
    assert rel(dw, e_dw) <= 1e-5     # fp32 dot products of exact 16-bit inputs


@pytest.mark.parametrize("F", [1, 8, 32])
def test_edge_dot_twin_against_oracle(F):
    rp, col, g = _graph(70 + F, 1800, 64)
    rng = np.random.default_rng(F)
    x = rng.standard_normal((1800, F)).astype(np.float32)
    dout = rng.standard_normal((1800, F)).astype(np.float32)
    dw = np.empty(g.E, np.float32)
    call("tgx_cpu_csr_edge_dot", p(g.rp), p(g.col), 64, g.plan.ref, p(x), p(dout), p(dw), 1800,
         1800, F, F32)
    assert rel(dw, ref.sum_bwd(rp, col, x, None, dout)[1]) <= 1e-5
    with pytest.raises(NotImplementedError, match="F <= 32"):
        call("tgx_cpu_csr_edge_dot", p(g.rp), p(g.col), 64, g.plan.ref, p(x), p(dout), p(dw),
             1800, 1800, 33, F32)


def test_sum_twin_of_an_edge_field_per_row():
    rp, col, g = _graph(9, 1500, 64)
    x = np.random.default_rng(9).standard_normal((g.E, 5)).astype(np.float32)
    out = np.empty((1500, 5), np.float32)
    call("tgx_cpu_csr_sum_fwd", p(g.rp), None, 64, g.plan.ref, p(x), None, p(out), 1500, g.E, 5,
         F32)
    assert rel(out, ref.sum_fwd(rp, np.arange(g.E), x)) <= 1e-5


# ---- GAT -------------------------------------------------------------------------------

@pytest.mark.parametrize("H,D", [(8, 32), (4, 64), (8, 64), (3, 64), (5, 8), (1, 4)])
@pytest.mark.parametrize("bits", [32, 64])
def test_gat_twin_against_oracle(H, D, bits):
    N = 2000
    rp, col, g = _graph(30 + H, N, bits)
    rng = np.random.default_rng(H * D)
    h = rng.standard_normal((N, H, D)).astype(np.float32)
    a_s = (0.1 * rng.standard_normal((H, D))).astype(np.float32)
    a_d = (0.1 * rng.standard_normal((H, D))).astype(np.float32)
    dout = rng.standard_normal((N, H, D)).astype(np.float32)
    out = np.empty_like(h)
    ns = np.empty((N, H, 4), np.float32)
    call("tgx_cpu_gat_fwd", p(g.rp), p(g.col), bits, g.plan.ref, p(h), p(h), p(a_s), p(a_d),
         0.2, p(out), p(ns), N, N, H, D, F32)
    e_out, e_lse = ref.gat_fwd(rp, col, h, a_s, a_d, 0.2)
    assert rel(out, e_out) <= 1e-5
    finite = np.isfinite(e_lse)
    assert (np.isfinite(ns[..., 0]) == finite).all()
    assert np.abs(ns[..., 0][finite] - e_lse[finite]).max() <= 1e-4
    assert rel(ns[..., 3], (h.astype(np.float64) * a_s).sum(-1)) <= 1e-5
    dh = np.empty_like(h)
    das = np.empty_like(a_s)
    dad = np.empty_like(a_d)
    call("tgx_cpu_gat_bwd", p(g.rp), p(g.col), bits, g.plan.ref, p(g.rpt), p(g.colt),
         p(g.perm), p(g.inv), g.plan_t.ref, p(h), p(h), p(a_s), p(a_d), 0.2, p(out), p(ns),
         p(dout), p(dh), p(dh), p(das), p(dad), N, N, g.E, H, D, F32)
    e_dh, e_das, e_dad = ref.gat_bwd(rp, col, h, a_s, a_d, 0.2, dout)
    assert rel(dh, e_dh) <= 1e-5
    assert rel(das, e_das) <= 1e-5
    assert rel(dad, e_dad) <= 1e-5


@pytest.mark.parametrize("kind", ["fp32", "bf16", "fp16"])
@pytest.mark.parametrize("bipartite", [False, True])
def test_gat_twin_element_types_and_bipartite(kind, bipartite):
    """The GAT twin with 16-bit elements (fp32 arithmetic, outputs rounded
    once: 2e-2) and with two feature tensors (1500 destinations, 2300
    sources) against the fp64 oracle on the type-rounded inputs."""
    dtype, code, tol = _DOT_DTYPES[kind]
    n_dst, n_src, H, D = 1500, 2300 if bipartite else 1500, 4, 32
    rp, col = skewed_csr(77, n_dst, n_src, mean_deg=8, hubs=(1200,), hot_src=5, hot_frac=0.2)
    g = HostGraph(rp, col, n_src, 64)
    rng = np.random.default_rng(3)
    mk = lambda n: torch.as_tensor(rng.standard_normal((n, H, D)), dtype=torch.float32).to(dtype)
    hs = mk(n_src)
    hd = mk(n_dst) if bipartite else hs
    dout = mk(n_dst)
    a_s = (0.1 * rng.standard_normal((H, D))).astype(np.float32)
    a_d = (0.1 * rng.standard_normal((H, D))).astype(np.float32)
    raw = (lambda t: np.ascontiguousarray(t.numpy())) if kind == "fp32" else _raw
    back = (lambda a: a.astype(np.float64)) if kind == "fp32" else \
        (lambda a: _from_raw(a, dtype))
    store = np.float32 if kind == "fp32" else np.int16
    rhs = raw(hs)
    rhd = raw(hd) if bipartite else rhs
    rg = raw(dout)
    out = np.zeros((n_dst, H, D), store)
    ns = np.empty((n_dst, H, 4), np.float32)
    call("tgx_cpu_gat_fwd", p(g.rp), p(g.col), 64, g.plan.ref, p(rhs), p(rhd), p(a_s), p(a_d),
         0.2, p(out), p(ns), n_dst, n_src, H, D, code)
    f = lambda t: t.double().numpy()
    e_out, _ = ref.gat_fwd(rp, col, f(hs), a_s, a_d, 0.2, h_dst=f(hd) if bipartite else None)
    assert rel(back(out), e_out) <= tol
    dhs = np.zeros((n_src, H, D), store)
    dhd = np.zeros((n_dst, H, D), store) if bipartite else dhs
    das, dad = np.empty_like(a_s), np.empty_like(a_d)
    call("tgx_cpu_gat_bwd", p(g.rp), p(g.col), 64, g.plan.ref, p(g.rpt), p(g.colt),
         p(g.perm), p(g.inv), g.plan_t.ref, p(rhs), p(rhd), p(a_s), p(a_d), 0.2, p(out), p(ns),
         p(rg), p(dhs), p(dhd), p(das), p(dad), n_dst, n_src, g.E, H, D, code)
    e = ref.gat_bwd_bipartite(rp, col, f(hs), f(hd), a_s, a_d, 0.2, f(dout))
    if bipartite:
        assert rel(back(dhs), e[0]) <= tol and rel(back(dhd), e[1]) <= tol
    else:
        assert rel(back(dhs), e[0] + e[1]) <= tol
    assert rel(das, e[2]) <= tol and rel(dad, e[3]) <= tol


def test_twin_results_do_not_depend_on_the_thread_count():
    N, H, D = 2000, 4, 32
    rp, col, g = _graph(41, N, 64)
    rng = np.random.default_rng(5)
    h = rng.standard_normal((N, H, D)).astype(np.float32)
    a = (0.1 * rng.standard_normal((2, H, D))).astype(np.float32)
    dout = rng.standard_normal((N, H, D)).astype(np.float32)
    runs = []
    for threads in (1, 3, 8):
        prev = _native.lib().tgx_cpu_set_threads(threads)
        try:
            out, ns = np.empty_like(h), np.empty((N, H, 4), np.float32)
            call("tgx_cpu_gat_fwd", p(g.rp), p(g.col), 64, g.plan.ref, p(h), p(h), p(a[0]),
                 p(a[1]), 0.2, p(out), p(ns), N, N, H, D, F32)
            dh, das, dad = np.empty_like(h), np.empty_like(a[0]), np.empty_like(a[1])
            call("tgx_cpu_gat_bwd", p(g.rp), p(g.col), 64, g.plan.ref, p(g.rpt), p(g.colt),
                 p(g.perm), p(g.inv), g.plan_t.ref, p(h), p(h), p(a[0]), p(a[1]), 0.2, p(out),
                 p(ns), p(dout), p(dh), p(dh), p(das), p(dad), N, N, g.E, H, D, F32)
            runs.append((out, dh, das, dad))
        finally:
            _native.lib().tgx_cpu_set_threads(prev)
    for r in runs[1:]:
        for x, y in zip(runs[0], r):
            assert np.array_equal(x, y)


# ---- dot-product attention (bf16, fp16, fp32) ----------------------------------------

_DOT_DTYPES = {"bf16": (torch.bfloat16, 0, 2e-2), "fp16": (torch.float16, 1, 2e-2),
               "fp32": (torch.float32, 2, 1e-5)}


@pytest.mark.parametrize("H,D", [(4, 64), (16, 64), (3, 64), (1, 8)])
@pytest.mark.parametrize("with_bias", [False, True])
@pytest.mark.parametrize("kind", ["bf16", "fp16", "fp32"])
def test_dot_twin_against_oracle(H, D, with_bias, kind):
    """The CPU twin of the dot-product entry points in each element type
    against the fp64 oracle on the type-rounded inputs: fp32 within 1e-5,
    the 16-bit types (one rounding of each output) within 2e-2."""
    dtype, code, tol = _DOT_DTYPES[kind]
    rp, col = rmat_csr(5, 10)
    N, E = rp.size - 1, col.size
    g = HostGraph(rp, col, N, 64)
    rng = np.random.default_rng(H + D)
    q, k, v, dout = (torch.as_tensor(rng.standard_normal((N, H, D)), dtype=torch.float32)
                     .to(dtype) for _ in range(4))
    bias = rng.standard_normal((E, H)).astype(np.float32) if with_bias else None
    f = lambda t: t.double().numpy()
    raw = (lambda t: np.ascontiguousarray(t.numpy())) if kind == "fp32" else _raw
    back = (lambda a: a.astype(np.float64)) if kind == "fp32" else \
        (lambda a: _from_raw(a, dtype))
    store = np.float32 if kind == "fp32" else np.int16
    scale = D ** -0.5
    out = np.zeros((N, H, D), store)
    ml = np.empty((N, H, 2), np.float32)
    rq, rk, rv, rg = raw(q), raw(k), raw(v), raw(dout)
    call("tgx_cpu_dot_attn_fwd", p(g.rp), p(g.col), 64, g.plan.ref, p(rq), p(rk), p(rv),
         p(bias), scale, p(out), p(ml), N, N, H, D, code)
    e_out, _ = ref.dot_fwd(rp, col, f(q), f(k), f(v), scale, bias)
    assert rel(back(out), e_out) <= tol
    dq, dk, dv = (np.zeros((N, H, D), store) for _ in range(3))
    dbias = np.empty((E, H), np.float32) if with_bias else None
    call("tgx_cpu_dot_attn_bwd", p(g.rp), p(g.col), 64, g.plan.ref, p(g.rpt), p(g.colt),
         p(g.perm), g.plan_t.ref, p(rq), p(rk), p(rv), p(bias), scale, p(out), p(ml), p(rg),
         p(dq), p(dk), p(dv), p(dbias), N, N, H, D, code)
    e = ref.dot_bwd(rp, col, f(q), f(k), f(v), scale, bias, f(dout))
    for got, want in zip((dq, dk, dv), e[:3]):
        assert rel(back(got), want) <= tol
    if with_bias:
        assert rel(dbias, e[3]) <= tol


# ---- dense attention over block-diagonal relations -------------------------------------

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("lane_major", [False, True])
@pytest.mark.parametrize("D", [32, 64])
def test_block_attention_twin_against_oracle(dtype, causal, lane_major, D):
    H = 2
    lengths = [70, 1, 130, 0, 33]
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    n = int(cu[-1])
    rng = np.random.default_rng(7)
    mk = lambda: torch.as_tensor(rng.standard_normal((n, H, D)), dtype=torch.float32).to(dtype)
    q, k, v, dout = mk(), mk(), mk(), mk()
    if lane_major:   # [H, n, D] storage viewed as [n, H, D]
        store = [t.transpose(0, 1).contiguous() for t in (q, k)]
        strides = (ctypes.c_int64 * 4)(D, n * D, D, n * D)
        rq, rk = _raw(store[0]), _raw(store[1])
    else:
        strides = (ctypes.c_int64 * 4)(H * D, D, H * D, D)
        rq, rk = _raw(q), _raw(k)
    # v shares k's strides.
    rv = _raw(v.transpose(0, 1).contiguous()) if lane_major else _raw(v)
    code = 0 if dtype == torch.bfloat16 else 1
    scale = D ** -0.5
    out = np.zeros((n, H, D), np.int16)
    lse = np.empty((n, H), np.float32)
    call("tgx_cpu_attn_fwd", p(cu), p(cu), len(lengths), int(causal), code, p(rq), p(rk), p(rv),
         strides, scale, 0.0, p(out), p(lse), n, n, H, D)
    f = lambda t: t.float().numpy()
    e_out, e_lse = ref.block_attention_fwd(cu, cu, f(q), f(k), f(v), scale, causal)
    assert rel(_from_raw(out, dtype), e_out) <= 2e-2
    ok = np.isfinite(e_lse)
    assert np.abs(lse[ok] - e_lse[ok]).max() <= 1e-3
    dq, dk, dv = (np.zeros((n, H, D), np.int16) for _ in range(3))
    delta = np.empty((n, H), np.float32)
    call("tgx_cpu_attn_bwd", p(cu), p(cu), len(lengths), int(causal), code, p(rq), p(rk), p(rv),
         strides, p(out), p(lse), p(_raw(dout)), scale, p(dq), p(dk), p(dv), p(delta), n, n, H,
         D)
    e = ref.block_attention_bwd(cu, cu, f(q), f(k), f(v), scale, causal, f(dout))
    for got, want in zip((dq, dk, dv), e):
        assert rel(_from_raw(got, dtype), want) <= 2e-2


# ---- argument and index checks -----------------------------------------------------------

def test_twin_checks_reject_bad_indices_and_plans():
    rp, col, g = _graph(3, 600, 64, hubs=(700,))
    x = np.ones((600, 4), np.float32)
    out = np.empty((600, 4), np.float32)
    bad = g.col.copy()
    bad[17] = 600
    with pytest.raises(RuntimeError, match="outside"):
        call("tgx_cpu_csr_sum_fwd", p(g.rp), p(bad), 64, g.plan.ref, p(x), None, p(out), 600,
             600, 4, F32)
    drop = g.rp.copy()
    drop[5] = drop[6] + 1
    with pytest.raises(RuntimeError, match="decreases"):
        call("tgx_cpu_csr_sum_fwd", p(drop), p(g.col), 64, g.plan.ref, p(x), None, p(out), 600,
             600, 4, F32)
    # A plan whose rows repeat, or whose chunk offsets miscount a split row.
    rows = g.plan.rows.copy()
    rows[1] = rows[0]
    twice = _native.RowPlan(*[getattr(g.plan.plan, f) for f, _ in _native.RowPlan._fields_])
    twice.rows_dev = p(rows)
    with pytest.raises(RuntimeError, match="twice"):
        call("tgx_cpu_csr_sum_fwd", p(g.rp), p(g.col), 64, ctypes.byref(twice), p(x), None,
             p(out), 600, 600, 4, F32)
    chunks = g.plan.chunks.copy()
    chunks[1:] += 1
    miscount = _native.RowPlan(*[getattr(g.plan.plan, f) for f, _ in _native.RowPlan._fields_])
    miscount.chunk_offsets_dev = p(chunks)
    miscount.n_chunks += 1
    with pytest.raises(RuntimeError, match="chunks"):
        call("tgx_cpu_csr_sum_fwd", p(g.rp), p(g.col), 64, ctypes.byref(miscount), p(x), None,
             p(out), 600, 600, 4, F32)
    # perm that is not a permutation.
    perm = g.perm.copy()
    perm[0] = perm[1]
    with pytest.raises(RuntimeError, match="permutation"):
        call("tgx_cpu_csr_sum_bwd", p(g.rpt), p(g.colt), p(perm), g.plan_t.ref, p(x), None,
             p(out), p(np.empty_like(x)), None, 600, 600, 4, F32)
    # Exact softmax only in the block-attention twin.
    cu = np.array([0, 64], np.int32)
    z = np.zeros((64, 1, 64), np.int16)
    with pytest.raises(NotImplementedError, match="exact softmax"):
        call("tgx_cpu_attn_fwd", p(cu), p(cu), 1, 1, 0, p(z), p(z), p(z),
             (ctypes.c_int64 * 4)(64, 64, 64, 64), 0.125, 0.5, p(z),
             p(np.empty((64, 1), np.float32)), 64, 64, 1, 64)


def _status(name, *args):
    return getattr(_native.lib(), name)(*args)


@pytest.mark.parametrize("H", [1, 2, 3, 8, 12])
@pytest.mark.parametrize("D", [2, 4, 6, 8, 12, 16, 32, 48, 64, 128, 256, 512, 1024])
def test_device_and_twin_reject_the_same_head_shapes(H, D):
    # Zero rows: the device entry points return after their shape and plan
    # checks, before any HIP call.
    empty = _native.RowPlan(0, 0, 0, 0, 0, WAVE_MAX, CHUNK, None, None)
    rp = np.zeros(1, np.int64)
    dummy = np.zeros(16, np.float32)
    gat_dev = _status("tgx_gat_fwd", p(rp), p(rp), 64, ctypes.byref(empty), p(dummy), p(dummy),
                      p(dummy), p(dummy), ctypes.c_float(0.2), p(dummy), p(dummy), 0, 0, H, D,
                      2, None, None, None)
    gat_cpu = _status("tgx_cpu_gat_fwd", p(rp), p(rp), 64, ctypes.byref(empty), p(dummy),
                      p(dummy), p(dummy), p(dummy), ctypes.c_float(0.2), p(dummy), p(dummy), 0,
                      0, H, D, 2)
    assert gat_dev == gat_cpu
    assert (gat_dev == 0) == (D % 4 == 0 and D <= 256 and (D // 4) & (D // 4 - 1) == 0)
    dot_dev = _status("tgx_dot_attn_fwd", p(rp), p(rp), 64, ctypes.byref(empty), p(dummy),
                      p(dummy), p(dummy), None, ctypes.c_float(1.0), p(dummy), p(dummy), 0, 0,
                      H, D, 0, None, None)
    dot_cpu = _status("tgx_cpu_dot_attn_fwd", p(rp), p(rp), 64, ctypes.byref(empty), p(dummy),
                      p(dummy), p(dummy), None, ctypes.c_float(1.0), p(dummy), p(dummy), 0, 0,
                      H, D, 0)
    assert dot_dev == dot_cpu
    assert (dot_dev == 0) == (D % 8 == 0 and D <= 512 and (D // 8) & (D // 8 - 1) == 0)

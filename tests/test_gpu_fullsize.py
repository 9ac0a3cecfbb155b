"""GPU checks at the benchmark configurations' full sizes.

The CPU oracle finishes the weighted sum (C1) at full size in seconds, so C1 is
compared with it directly.  The attention configurations are too large for the
fp64 oracle; they are checked through properties that hold at any size:

* softmax weights sum to one: with a value field of ones every non-empty row
  gives 1 (empty rows give 0);
* with all scores equal (GAT with a_src = a_dst = 0) the output is the
  neighbour mean and dh is the mean's adjoint;
* each output row is a convex combination of its neighbours' value rows;
* the softmax Jacobian's rows sum to zero, so per destination row the score
  gradients add up to 0 and the value gradients summed over all sources equal
  the sum of dout over the non-empty rows.  The bf16 paths form the backward's
  row term delta = <dout, out> from the bf16-rounded output (as FlashAttention
  does), so there a row's score gradients add up to a residual bounded by
  2^-8 <|dout|, |out|> rather than to 0, and the key gradients summed over all
  keys equal scale * sum_i q_i * (row i's residual);
* a causal sequence's first token sees only itself: its output is its value;
* reruns are bit-identical (no floating-point atomics).

Tolerances: fp32 paths 1e-5 relative (max-norm) where a reference value
exists, bf16 paths 2e-2; sums that should vanish are bounded relative to the
sum of the magnitudes of their terms (fp32 1e-4, bf16 1e-2).
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import tiga as tg
from oracle import ref

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
SEED = 20260821


@pytest.fixture(autouse=True)
def _strict():
    tg.config.strict = True
    yield
    tg.config.strict = False


def rel_err(actual, expected):
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    return float(np.abs(a - e).max() / max(np.abs(e).max(), 1e-30))


def vanishing(total, magnitude, tol):
    """|total| <= tol * magnitude elementwise (both fp64 tensors)."""
    return bool((total.abs() <= tol * magnitude + 1e-30).all())


# ---- graphs (seeded, on the GPU) ---------------------------------------------

def fixed_degree(n, degree, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    col = torch.randint(0, n, (n, degree), device=DEV, generator=g)
    col, _ = torch.sort(col, dim=1)
    return torch.arange(n + 1, dtype=torch.int64, device=DEV) * degree, col.reshape(-1)


def poisson_self_loop(n, mean, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    deg = torch.poisson(torch.full((n,), float(mean), device=DEV), generator=g).to(torch.int64)
    rows = torch.repeat_interleave(torch.arange(n, device=DEV), deg)
    cols = torch.randint(0, n, (int(deg.sum().item()),), device=DEV, generator=g)
    ar = torch.arange(n, device=DEV)
    keys, _ = torch.sort(torch.cat([rows * n + cols, ar * n + ar]))
    row_ptr = torch.zeros(n + 1, dtype=torch.int64, device=DEV)
    row_ptr[1:] = torch.cumsum(deg + 1, 0)
    return row_ptr, keys % n


def rmat(scale, edge_factor, seed, probs=(0.57, 0.19, 0.19, 0.05)):
    g = torch.Generator(device=DEV).manual_seed(seed)
    n, m = 1 << scale, edge_factor << scale
    a, b, c, _ = probs
    row = torch.zeros(m, dtype=torch.int64, device=DEV)
    col = torch.zeros(m, dtype=torch.int64, device=DEV)
    for level in range(scale):
        r = torch.rand(m, device=DEV, generator=g)
        row |= (r >= a + b).to(torch.int64) << level
        col |= (((r >= a) & (r < a + b)) | (r >= a + b + c)).to(torch.int64) << level
    keys = torch.unique(row * n + col)
    row_ptr = torch.zeros(n + 1, dtype=torch.int64, device=DEV)
    row_ptr[1:] = torch.cumsum(torch.bincount(keys // n, minlength=n), 0)
    return row_ptr, keys % n


def row_sums(values, row_ptr):
    """Per-row sums of an edge-ordered tensor, fp64."""
    return torch.segment_reduce(values.double(), "sum", offsets=row_ptr, axis=0)


# ---- C1: weighted sum, 100k x 16, F = 64, fp32 -----------------------------------

class WeightedSum(tg.MessagePassing):
    reducer = tg.sum()

    def edge(self, src, dst, edge):
        return edge.weight * src.x


def test_c1_full_size_against_oracle():
    print("c1 full size: 100000 x 16, F=64", flush=True)
    N, deg, F_ = 100_000, 16, 64
    row_ptr, col = fixed_degree(N, deg, SEED)
    g = torch.Generator(device=DEV).manual_seed(SEED + 1)
    x = torch.randn(N, F_, device=DEV, generator=g).requires_grad_(True)
    w = torch.rand(col.numel(), 1, device=DEV, generator=g).requires_grad_(True)
    dout = torch.randn(N, F_, device=DEV, generator=g)
    kernel = WeightedSum()
    out = kernel(graph=tg.Graph.from_csr(row_ptr, col, num_src=N), src={"x": x}, dst={},
                 edge={"weight": w})
    assert kernel.last_variant.backend == "hip"
    out.backward(dout)
    rp, c = row_ptr.cpu().numpy(), col.cpu().numpy()
    xh, wh, dh = x.detach().cpu().numpy(), w.detach().cpu().numpy(), dout.cpu().numpy()
    assert rel_err(out.detach().cpu(), ref.sum_fwd(rp, c, xh, wh)) <= 1e-5
    e_dx, e_dw = ref.sum_bwd(rp, c, xh, wh, dh)
    assert rel_err(x.grad.cpu(), e_dx) <= 1e-5
    assert rel_err(w.grad.cpu().reshape(-1), np.asarray(e_dw).reshape(-1)) <= 1e-5


# ---- C2: GAT additive, 1M nodes, Poisson(16) + self-loop, H = 8, D = 32, fp32 ---

def gat(a_src, a_dst, slope=0.2):
    class GAT(tg.MessagePassing):
        reducer = tg.online_softmax()

        def edge(self, src, dst, edge):
            s = F.leaky_relu((src.h * a_src).sum(-1) + (dst.h * a_dst).sum(-1), slope)
            return self.reducer(s, src.h)

    return GAT()


@pytest.fixture(scope="module")
def c2_graph():
    row_ptr, col = poisson_self_loop(1_000_000, 16.0, SEED)
    return row_ptr, col, tg.Graph.from_csr(row_ptr, col, num_src=row_ptr.numel() - 1)


def test_c2_full_size_equal_scores_give_neighbour_mean(c2_graph):
    print("c2 full size: a = 0, neighbour mean", flush=True)
    row_ptr, col, graph = c2_graph
    N, H, D = row_ptr.numel() - 1, 8, 32
    g = torch.Generator(device=DEV).manual_seed(SEED + 1)
    h = torch.randn(N, H, D, device=DEV, generator=g).requires_grad_(True)
    zero = torch.zeros(H, D, device=DEV)
    dout = torch.randn(N, H, D, device=DEV, generator=g)
    kernel = gat(zero, zero)
    out = kernel(graph=graph, src={"h": h}, dst={"h": h})
    assert kernel.last_variant.backend == "hip"
    out.backward(dout)
    deg = (row_ptr[1:] - row_ptr[:-1]).to(torch.float64)
    hd = h.detach().reshape(N, H * D)
    mean = torch.segment_reduce(hd[col], "sum", offsets=row_ptr, axis=0).double()
    mean /= deg[:, None]
    assert rel_err(out.detach().reshape(N, -1).cpu(), mean.cpu()) <= 1e-5
    # dh[j] = sum over edges j -> i of dout[i] / deg(i) (the scores do not depend
    # on h when a = 0).
    dst = torch.repeat_interleave(torch.arange(N, device=DEV), row_ptr[1:] - row_ptr[:-1])
    msg = (dout.reshape(N, -1).double() / deg[:, None])[dst]
    e_dh = torch.zeros(N, H * D, dtype=torch.float64, device=DEV).index_add_(0, col, msg)
    assert rel_err(h.grad.reshape(N, -1).cpu(), e_dh.cpu()) <= 1e-5


def test_c2_full_size_convexity_and_reruns(c2_graph):
    print("c2 full size: random a, convex hull and reruns", flush=True)
    row_ptr, col, graph = c2_graph
    N, H, D = row_ptr.numel() - 1, 8, 32
    g = torch.Generator(device=DEV).manual_seed(SEED + 2)
    h = torch.randn(N, H, D, device=DEV, generator=g).requires_grad_(True)
    a_src = (0.1 * torch.randn(H, D, device=DEV, generator=g)).requires_grad_(True)
    a_dst = (0.1 * torch.randn(H, D, device=DEV, generator=g)).requires_grad_(True)
    dout = torch.randn(N, H, D, device=DEV, generator=g)
    runs = []
    for _ in range(2):
        h.grad = a_src.grad = a_dst.grad = None
        kernel = gat(a_src, a_dst)
        out = kernel(graph=graph, src={"h": h}, dst={"h": h})
        assert kernel.last_variant.backend == "hip"
        out.backward(dout)
        runs.append([t.detach().clone() for t in (out, h.grad, a_src.grad, a_dst.grad)])
    for a, b in zip(*runs):
        assert torch.equal(a, b)
    out = runs[0][0].reshape(N, -1)
    assert torch.isfinite(out).all() and all(torch.isfinite(t).all() for t in runs[0][1:])
    gathered = h.detach().reshape(N, -1)[col]
    lo = torch.segment_reduce(gathered, "min", offsets=row_ptr, axis=0)
    hi = torch.segment_reduce(gathered, "max", offsets=row_ptr, axis=0)
    del gathered
    slack = 1e-5 * (hi - lo).abs() + 1e-6
    assert bool(((out >= lo - slack) & (out <= hi + slack)).all())


# ---- C3/C4: dot-product attention, R-MAT scale 21, H = 4, D = 64, bf16 -----------

class DotAttention(tg.MessagePassing):
    reducer = tg.online_softmax()

    def edge(self, src, dst, edge, scale):
        return self.reducer((src.k * dst.q).sum(dim=-1) * scale + edge.bias, src.v)


def test_c3_c4_full_size_softmax_identities():
    print("c3/c4 full size: R-MAT scale 21", flush=True)
    row_ptr, col = rmat(21, 16, SEED)
    N, E, H, D = row_ptr.numel() - 1, col.numel(), 4, 64
    graph = tg.Graph.from_csr(row_ptr, col, num_src=N)
    g = torch.Generator(device=DEV).manual_seed(SEED + 1)
    mk = lambda: torch.randn(N, H, D, device=DEV, generator=g).to(torch.bfloat16)
    q, k, v = (mk().requires_grad_(True) for _ in range(3))
    bias = torch.randn(E, H, device=DEV, generator=g).requires_grad_(True)
    dout = mk()
    nonempty = row_ptr[1:] > row_ptr[:-1]
    kernel = DotAttention()
    # Weights sum to one: a value field of ones gives 1 on every non-empty row.
    ones = torch.ones(N, H, D, device=DEV, dtype=torch.bfloat16)
    with torch.no_grad():
        o1 = kernel(graph=graph, src={"k": k, "v": ones}, dst={"q": q}, edge={"bias": bias},
                    scale=D ** -0.5)
    assert kernel.last_variant.backend == "hip"
    assert float((o1[nonempty].float() - 1).abs().max()) <= 2e-2
    assert torch.count_nonzero(o1[~nonempty]).item() == 0
    runs = []
    for _ in range(2):
        q.grad = k.grad = v.grad = bias.grad = None
        out = kernel(graph=graph, src={"k": k, "v": v}, dst={"q": q}, edge={"bias": bias},
                     scale=D ** -0.5)
        out.backward(dout)
        runs.append([t.detach().clone() for t in (out, q.grad, k.grad, v.grad, bias.grad)])
    for a, b in zip(*runs):
        assert torch.equal(a, b)
    out, dq, dk, dv, dbias = runs[0]
    for t in (out, dq, dk, dv, dbias):
        assert torch.isfinite(t.float()).all()
    # Per row the score gradients add up to the bf16 rounding residual of delta.
    resid = row_sums(dbias, row_ptr)                                   # [N, H]
    bound = 2.0 ** -8 * (dout.double().abs() * out.double().abs()).sum(-1)
    assert vanishing(resid, row_sums(dbias.abs(), row_ptr) * 1e-4 + bound, 1.0)
    # sum_j dk[j] = scale * sum_i q[i] * (row i's score-gradient sum).
    e_dk = D ** -0.5 * (q.detach().double() * resid[:, :, None]).sum(0)
    assert vanishing(dk.double().sum(0) - e_dk, dk.double().abs().sum(0), 1e-2)
    # sum_j dv[j] = sum over non-empty rows of dout (each row's weights sum to one).
    dsum = dout.double()[nonempty].sum(0)
    assert vanishing(dv.double().sum(0) - dsum, dout.double().abs().sum(0), 1e-3)


# ---- C5: varlen causal attention, 32 sequences U[512, 4096], H = 16, D = 128 ----

class VarlenAttention(tg.MessagePassing):
    reducer = tg.online_softmax()

    def edge(self, src, dst, edge, scale):
        return self.reducer((src.key * dst.query).sum(dim=-1) * scale, src.value)


def test_c5_full_size_causal_identities():
    rng = np.random.default_rng(SEED)
    lengths = rng.integers(512, 4097, size=32)
    print(f"c5 full size: {int(lengths.sum())} tokens", flush=True)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lengths)]), dtype=torch.int64, device=DEV)
    T, H, D = int(lengths.sum()), 16, 128
    g = torch.Generator(device=DEV).manual_seed(SEED + 1)
    mk = lambda: torch.randn(T, H, D, device=DEV, generator=g).to(torch.bfloat16)
    q, k, v = (mk().requires_grad_(True) for _ in range(3))
    dout = mk()
    graph = tg.Graph.cu_seqlens(cu, causal=True)
    kernel = VarlenAttention()
    runs = []
    for _ in range(2):
        q.grad = k.grad = v.grad = None
        out = kernel(graph=graph, src={"key": k, "value": v}, dst={"query": q}, scale=D ** -0.5)
        assert kernel.last_variant.backend == "hip"
        out.backward(dout)
        runs.append([t.detach().clone() for t in (out, q.grad, k.grad, v.grad)])
    for a, b in zip(*runs):
        assert torch.equal(a, b)
    out, dq, dk, dv = runs[0]
    for t in (out, dq, dk, dv):
        assert torch.isfinite(t.float()).all()
    first = cu[:-1]
    # A sequence's first token attends only to itself.
    assert torch.equal(out[first], v.detach()[first])
    # Per sequence: the values' gradients sum to sum(dout); the keys' gradients
    # to scale * sum_q q * (row q's score-gradient sum), which the bf16 rounding
    # of out in delta bounds by 2^-8 <|dout_q|, |out_q|>.
    seg = lambda t: torch.segment_reduce(t.double(), "sum", offsets=cu, axis=0)
    assert vanishing(seg(dv) - seg(dout), seg(dout.abs()), 1e-3)
    row_bound = 2.0 ** -8 * (dout.double().abs() * out.double().abs()).sum(-1)   # [T, H]
    dk_bound = D ** -0.5 * seg(q.detach().double().abs() * row_bound[:, :, None])
    assert vanishing(seg(dk), 1e-2 * seg(dk.abs()) + dk_bound, 1.0)


# ---- nn-scored attention: 131072 nodes, ~4.0M edges, net 19-16-1, fp32 -------------

def test_nn_full_size_softmax_identities():
    from torch import nn

    print("nn full size: 131072 nodes", flush=True)
    N = 131072
    row_ptr, col = poisson_self_loop(N, 29.6, SEED)
    graph = tg.Graph.from_csr(row_ptr, col, num_src=N)
    g = torch.Generator(device=DEV).manual_seed(SEED + 1)
    pos = torch.rand(N, 3, device=DEV, generator=g)
    x = torch.randn(N, 8, device=DEV, generator=g).requires_grad_(True)
    disp = (pos[col] - pos[graph.destination_index()]).requires_grad_(True)
    ones = torch.ones(N, 8, device=DEV)
    torch.manual_seed(SEED)
    net = nn.Sequential(nn.Linear(19, 16), nn.LeakyReLU(0.2), nn.Linear(16, 1)).to(DEV)
    dout = torch.randn(N, 8, device=DEV, generator=g)

    class GAT(tg.MessagePassing):
        reducer = tg.online_softmax()

        def __init__(self):
            super().__init__()
            self.attn = tg.nn.trace(net)

        def edge(self, src, dst, edge):
            return self.reducer(self.attn(edge.displacement, src.x, dst.x), src.value)

    kernel = GAT()
    with torch.no_grad():
        o1 = kernel(graph=graph, src={"x": x, "value": ones}, dst={"x": x},
                    edge={"displacement": disp})
    assert kernel.last_variant.backend == "hip"
    assert float((o1 - 1).abs().max()) <= 1e-5
    runs = []
    for _ in range(2):
        x.grad = disp.grad = None
        net.zero_grad(set_to_none=True)
        out = kernel(graph=graph, src={"x": x, "value": x}, dst={"x": x},
                     edge={"displacement": disp})
        out.backward(dout)
        runs.append([t.detach().clone() for t in
                     (out, x.grad, disp.grad, *(p.grad for p in net.parameters()))])
    for a, b in zip(*runs):
        assert torch.equal(a, b)
    assert all(torch.isfinite(t).all() for t in runs[0])
    # The last layer's bias gradient is the sum of all score gradients, which
    # vanishes row by row; its weight gradient (sum of ds * hidden) does not.
    db_last, dw_last = net[2].bias.grad.double(), net[2].weight.grad.double()
    assert float(db_last.abs().max()) <= 1e-2 * float(dw_last.abs().max())

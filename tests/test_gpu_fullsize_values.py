"""GPU value parity at the benchmark configurations' full sizes, and against
the reference's own bf16 arithmetic.

* C2 (GAT fp32, 1M nodes, 17M edges): out, dh, da_src and da_dst against
  the row-chunked float64 restatement (oracle/chunked.py, pinned against
  oracle/ref.py in tests/test_oracle.py), max|gpu - oracle| <= 1e-5 *
  max|oracle| per tensor.  da_src / da_dst are 17M-edge reductions.
  LeakyReLU's derivative jumps at z = 0: among 136M (edge, head) pairs a
  few have fp32 and fp64 values of z on opposite sides of 0, where the two
  derivatives differ by (1 - slope) * dscore.  The checker takes the piece
  from the kernel's own fp32 z (its saved node state holds both halves of
  z; the kernel adds them in fp32, which the checker repeats exactly), after
  checking those halves against fp64 math; the count of such pairs is
  printed.
* C3 (dot-product bf16, R-MAT scale 21): out on every row above 512 edges
  (the split hub rows) and on a seeded sample of other rows, 2e-2.
* C4 (its fused backward): dq, dk, dv and dbias over the whole graph, 2e-2.
* C5 (varlen causal, 32 sequences of U[512, 4096] tokens, bf16): out, dq, dk
  and dv of the longest sequence and two seeded others, against the
  query-chunked float64 per-sequence attention, 2e-2.
* nn-scored attention (the reference's GAT example shape, 131072 nodes,
  4.0M edges, fp32, value = the source field): out, the field gradients and
  the weight gradients against the float64 Torch checker
  (oracle/chunked.nn_attention), 1e-5, away from LeakyReLU's kink.
* bf16 arithmetic: on an R-MAT scale-12 graph the HIP dot-product forward
  and backward against the reference's eager path run in bf16 on the CPU
  (oracle/eager_torch.dot_reference: bf16 q*k products and sums, fp32 bias
  and softmax accumulation, bf16 output) and against float64 math.  Against
  float64 the bar is 2e-2.  Against the reference's bf16 results it is 2e-2
  plus that result's own distance from float64: the reference's autograd
  sums dk and dv into bf16 leaves (index_add in bf16), which over a hub's
  many out-edges moves it several 1e-2 from exact math, while these kernels
  accumulate in fp32.

The float64 checker runs with Torch's own float64 kernels on the GPU (the
CPU would take minutes at these sizes); the bf16 inputs enter it exactly.
Beside each max-norm error the tests print element-wise relative errors
(median, 99.9th percentile, maximum over elements above 1e-3 of the
largest), so small elements are visible too.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import tiga as tg
from oracle import chunked, eager_torch, ref

from test_gpu_fullsize import DotAttention, gat, poisson_self_loop, rmat

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
SEED = 20260822


@pytest.fixture(autouse=True)
def _strict():
    tg.config.strict = True
    yield
    tg.config.strict = False


def rel(actual, expected) -> float:
    a, e = actual.double(), expected.double()
    return float((a - e).abs().max() / e.abs().max().clamp_min(1e-300))


def elementwise(actual, expected) -> str:
    """Element-wise relative errors |a - e| / |e|, printed beside the
    max-norm bound: median, 99.9th percentile and maximum over the elements
    with |e| >= 1e-3 max|e| (a strided sample of at most 4M of them)."""
    a, e = actual.detach().double().flatten(), expected.detach().double().flatten()
    keep = e.abs() >= 1e-3 * e.abs().max()
    r = (a - e).abs()[keep] / e.abs()[keep]
    if r.numel() == 0:
        return "elementwise: no elements"
    sample = r[::max(1, r.numel() // (1 << 22))].float()
    p50, p999 = torch.quantile(sample, torch.tensor([0.5, 0.999], device=sample.device))
    return f"elementwise p50 {float(p50):.2e} p99.9 {float(p999):.2e} max {float(r.max()):.2e}"


def test_c2_full_size_values_against_float64():
    print("c2 full size values: 1M nodes, fp64 checker", flush=True)
    row_ptr, col = poisson_self_loop(1_000_000, 16.0, SEED)
    N, H, D = row_ptr.numel() - 1, 8, 32
    graph = tg.Graph.from_csr(row_ptr, col, num_src=N)
    g = torch.Generator(device=DEV).manual_seed(SEED + 1)
    h = torch.randn(N, H, D, device=DEV, generator=g).requires_grad_(True)
    a_src = (0.1 * torch.randn(H, D, device=DEV, generator=g)).requires_grad_(True)
    a_dst = (0.1 * torch.randn(H, D, device=DEV, generator=g)).requires_grad_(True)
    dout = torch.randn(N, H, D, device=DEV, generator=g)
    kernel = gat(a_src, a_dst)
    out = kernel(graph=graph, src={"h": h}, dst={"h": h})
    assert kernel.last_variant.backend == "hip"
    # The kernel's own fp32 halves of z (node state slots 3 and 2: a_src.h,
    # a_dst.h), read before the backward reuses slot 1.  The node state is
    # the last tensor the GAT autograd function saves.
    node_state = out.grad_fn.saved_tensors[-1]
    assert tuple(node_state.shape) == (N, H, 4)
    branch = (node_state[..., 3].clone(), node_state[..., 2].clone())
    out.backward(dout)
    torch.cuda.synchronize()
    d = lambda t: t.detach().double()
    # The halves agree with fp64 math to fp32 rounding.
    assert rel(branch[0], (d(h) * d(a_src)).sum(-1)) <= 1e-6
    assert rel(branch[1], (d(h) * d(a_dst)).sum(-1)) <= 1e-6
    e_out, _ = chunked.gat_fwd(row_ptr, col, d(h), d(a_src), d(a_dst), 0.2)
    print(f"c2 out {rel(out.detach(), e_out):.3e}, {elementwise(out, e_out)}", flush=True)
    assert rel(out.detach(), e_out) <= 1e-5
    del e_out
    stats = {}
    e_dh, e_das, e_dad = chunked.gat_bwd(row_ptr, col, d(h), d(a_src), d(a_dst), 0.2, d(dout),
                                         branch=branch, stats=stats)
    errs = {"dh": rel(h.grad, e_dh), "da_src": rel(a_src.grad, e_das),
            "da_dst": rel(a_dst.grad, e_dad)}
    print(f"c2 relative errors {errs}; (edge, head) pairs whose fp32 and fp64 z straddle "
          f"the LeakyReLU kink: {stats['kink_flips']}; dh {elementwise(h.grad, e_dh)}",
          flush=True)
    assert all(e <= 1e-5 for e in errs.values()), errs


@pytest.fixture(scope="module")
def c34():
    row_ptr, col = rmat(21, 16, SEED)
    N, E, H, D = row_ptr.numel() - 1, col.numel(), 4, 64
    g = torch.Generator(device=DEV).manual_seed(SEED + 1)
    mk = lambda: torch.randn(N, H, D, device=DEV, generator=g).to(torch.bfloat16)
    q, k, v = (mk().requires_grad_(True) for _ in range(3))
    bias = torch.randn(E, H, device=DEV, generator=g).requires_grad_(True)
    dout = mk()
    return row_ptr, col, tg.Graph.from_csr(row_ptr, col, num_src=N), q, k, v, bias, dout


def test_c3_full_size_hub_rows_and_a_sample_against_float64(c34):
    row_ptr, col, graph, q, k, v, bias, _ = c34
    D = q.shape[2]
    kernel = DotAttention()
    with torch.no_grad():
        out = kernel(graph=graph, src={"k": k, "v": v}, dst={"q": q}, edge={"bias": bias},
                     scale=D ** -0.5)
    assert kernel.last_variant.backend == "hip"
    deg = (row_ptr[1:] - row_ptr[:-1]).cpu()
    hubs = torch.nonzero(deg > 512).flatten()
    rng = np.random.default_rng(SEED)
    others = torch.nonzero((deg > 0) & (deg <= 512)).flatten().numpy()
    sample = rng.choice(others, size=min(20000, others.size), replace=False)
    rows = np.unique(np.concatenate([hubs.numpy(), sample]))
    print(f"c3 full size values: {hubs.numel()} hub rows + {sample.size} sampled rows",
          flush=True)
    d = lambda t: t.detach().double()
    e_out, _ = chunked.dot_fwd(row_ptr, col, d(q), d(k), d(v), D ** -0.5, d(bias), rows=rows)
    sel = torch.as_tensor(rows, device=DEV)
    err_hub = rel(out[hubs.to(DEV)], e_out[hubs.to(DEV)])
    err_all = rel(out[sel], e_out[sel])
    print(f"c3 relative errors hub {err_hub:.3e} sampled {err_all:.3e}", flush=True)
    assert err_hub <= 2e-2 and err_all <= 2e-2


def test_c4_full_size_gradients_against_float64(c34):
    print("c4 full size values: dq, dk, dv, dbias", flush=True)
    row_ptr, col, graph, q, k, v, bias, dout = c34
    D = q.shape[2]
    kernel = DotAttention()
    out = kernel(graph=graph, src={"k": k, "v": v}, dst={"q": q}, edge={"bias": bias},
                 scale=D ** -0.5)
    assert kernel.last_variant.backend == "hip"
    q.grad = k.grad = v.grad = bias.grad = None
    out.backward(dout)
    torch.cuda.synchronize()
    d = lambda t: t.detach().double()
    want = chunked.dot_bwd(row_ptr, col, d(q), d(k), d(v), D ** -0.5, d(bias), d(dout))
    errs = {n: rel(g, w) for n, g, w in zip(("dq", "dk", "dv", "dbias"),
                                            (q.grad, k.grad, v.grad, bias.grad), want)}
    print(f"c4 relative errors {errs}", flush=True)
    for n, g, w in zip(("dq", "dk", "dv", "dbias"), (q.grad, k.grad, v.grad, bias.grad), want):
        print(f"  {n} {elementwise(g, w)}", flush=True)
    assert all(e <= 2e-2 for e in errs.values()), errs


def test_c5_full_size_sequences_against_float64():
    """C5 as the bench runs it (32 sequences of U[512, 4096] tokens, H = 16,
    D = 128, bf16, the bench's seed): out, dq, dk and dv of the longest
    sequence and of two seeded others against the query-chunked float64
    per-sequence causal attention (oracle/chunked.causal_sequence), 2e-2."""
    seed = 20260821                           # bench.py's default seed
    rng = np.random.default_rng(seed)
    lengths = rng.integers(512, 4097, size=32)
    cu_host = np.concatenate([[0], np.cumsum(lengths)])
    T, H, D = int(lengths.sum()), 16, 128
    picks = [int(np.argmax(lengths))]
    others = [b for b in range(32) if b != picks[0]]
    picks += [int(b) for b in np.random.default_rng(seed + 2).choice(others, 2, replace=False)]
    print(f"c5 full size values: {T} tokens, sequences {picks} of lengths "
          f"{[int(lengths[b]) for b in picks]}", flush=True)
    cu = torch.tensor(cu_host, dtype=torch.int64, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(seed + 1)
    mk = lambda: torch.randn(T, H, D, device=DEV, generator=g).to(torch.bfloat16)
    q, k, v = (mk().requires_grad_(True) for _ in range(3))
    dout = mk()
    from test_gpu_fullsize import VarlenAttention
    kernel = VarlenAttention()
    out = kernel(graph=tg.Graph.cu_seqlens(cu, causal=True), src={"key": k, "value": v},
                 dst={"query": q}, scale=D ** -0.5)
    assert kernel.last_variant.backend == "hip"
    out.backward(dout)
    torch.cuda.synchronize()
    got = (out.detach(), q.grad, k.grad, v.grad)
    d = lambda t: t.detach().double()
    worst = {}
    for b in picks:
        s0, s1 = int(cu_host[b]), int(cu_host[b + 1])
        e_out, _, e_dq, e_dk, e_dv = chunked.causal_sequence(
            d(q[s0:s1]), d(k[s0:s1]), d(v[s0:s1]), D ** -0.5, d(dout[s0:s1]))
        for name, gpu, want in zip(("out", "dq", "dk", "dv"), got, (e_out, e_dq, e_dk, e_dv)):
            err = rel(gpu[s0:s1], want)
            worst[name] = max(worst.get(name, 0.0), err)
            print(f"  sequence {b} (L={s1 - s0}) {name}: {err:.3e}, "
                  f"{elementwise(gpu[s0:s1], want)}", flush=True)
        del e_out, e_dq, e_dk, e_dv
    assert all(e <= 2e-2 for e in worst.values()), worst


@pytest.mark.parametrize("with_bias", [False, True])
def test_dot_against_the_reference_bf16_arithmetic(with_bias):
    print(f"bf16 reference arithmetic, R-MAT scale 12, bias={with_bias}", flush=True)
    row_ptr, col = rmat(12, 16, SEED + 7)
    N, E, H, D = row_ptr.numel() - 1, col.numel(), 4, 64
    graph = tg.Graph.from_csr(row_ptr, col, num_src=N)
    g = torch.Generator(device=DEV).manual_seed(SEED + 8)
    mk = lambda: torch.randn(N, H, D, device=DEV, generator=g).to(torch.bfloat16)
    q, k, v = (mk().requires_grad_(True) for _ in range(3))
    bias = torch.randn(E, H, device=DEV, generator=g).requires_grad_(with_bias)
    dout = mk()

    class Plain(tg.MessagePassing):
        reducer = tg.online_softmax()

        def edge(self, src, dst, edge, scale):
            return self.reducer((src.k * dst.q).sum(dim=-1) * scale, src.v)

    kernel = DotAttention() if with_bias else Plain()
    fields = {"edge": {"bias": bias}} if with_bias else {}
    out = kernel(graph=graph, src={"k": k, "v": v}, dst={"q": q}, scale=D ** -0.5, **fields)
    assert kernel.last_variant.backend == "hip"
    out.backward(dout)
    got = [out.detach(), q.grad, k.grad, v.grad] + ([bias.grad] if with_bias else [])
    cpu = lambda t: t.detach().cpu()
    rp, c = row_ptr.cpu(), col.cpu()
    b = cpu(bias) if with_bias else None
    eager = eager_torch.dot_reference(rp, c, cpu(q), cpu(k), cpu(v), b, D ** -0.5, cpu(dout))
    f64 = lambda t: t.detach().double().cpu().numpy()
    e_out, _ = ref.dot_fwd(rp.numpy(), c.numpy(), f64(q), f64(k), f64(v), D ** -0.5,
                           None if b is None else f64(b))
    e_grads = ref.dot_bwd(rp.numpy(), c.numpy(), f64(q), f64(k), f64(v), D ** -0.5,
                          None if b is None else f64(b), f64(dout))
    exact = [e_out, *e_grads[:3]] + ([e_grads[3]] if with_bias else [])
    for name, gpu, e16, e64 in zip(("out", "dq", "dk", "dv", "dbias"), got, eager, exact):
        e64 = torch.as_tensor(e64)
        err16 = rel(gpu.cpu(), e16)
        err64 = rel(gpu.cpu(), e64)
        own = rel(e16, e64)   # the reference's bf16 path against exact math
        print(f"  {name}: vs reference bf16 {err16:.3e}, vs fp64 {err64:.3e}; reference bf16 "
              f"vs fp64 {own:.3e}", flush=True)
        assert err64 <= 2e-2, name
        assert err16 <= 2e-2 + own, name


# ---- nn-scored attention at the bench's size: 131072 nodes, ~4.0M edges --------

def test_nn_full_size_values_against_float64():
    """The reference's GAT example shape (score net Linear(19, 16) ->
    LeakyReLU(0.2) -> Linear(16, 1) over [displacement | x_src | x_dst], value
    x_src, so the backward folds the value gradient into the source field's
    rows) at the bench configuration, against the float64 Torch checker
    (oracle/chunked.nn_attention, pinned against ref.nn_attention_fwd/bwd):
    out and the gradients of x and the displacement within 1e-5 of the
    largest element (away from LeakyReLU's kink, below), the weight and bias
    gradients (sums over all 4.0M edges) within 1e-5 plus, for the hidden
    layer, the kink's bounded share."""
    from torch import nn

    print("nn full size values: 131072 nodes", flush=True)
    N = 131072
    row_ptr, col = poisson_self_loop(N, 29.6, SEED)
    graph = tg.Graph.from_csr(row_ptr, col, num_src=N)
    g = torch.Generator(device=DEV).manual_seed(SEED + 3)
    pos = torch.rand(N, 3, device=DEV, generator=g)
    x = torch.randn(N, 8, device=DEV, generator=g).requires_grad_(True)
    disp = (pos[col] - pos[graph.destination_index()]).requires_grad_(True)
    torch.manual_seed(SEED + 3)
    net = nn.Sequential(nn.Linear(19, 16), nn.LeakyReLU(0.2), nn.Linear(16, 1)).to(DEV)
    dout = torch.randn(N, 8, device=DEV, generator=g)

    class GAT(tg.MessagePassing):
        reducer = tg.online_softmax()

        def __init__(self):
            super().__init__()
            self.attn = tg.nn.trace(net)

        def edge(self, src, dst, edge):
            return self.reducer(self.attn(edge.displacement, src.x, dst.x), src.x)

    kernel = GAT()
    out = kernel(graph=graph, src={"x": x}, dst={"x": x}, edge={"displacement": disp})
    assert kernel.last_variant.backend == "hip"
    out.backward(dout)
    d64 = lambda t: t.detach().double()
    layers = [(d64(net[0].weight), d64(net[0].bias), "leaky_relu", 0.2),
              (d64(net[2].weight), d64(net[2].bias), "identity", 0.0)]
    e_out, (e_disp, e_src, e_dst), e_val, e_layers, hidden = chunked.nn_attention(
        row_ptr.long(), col.long(), [("edge", d64(disp)), ("src", d64(x)), ("dst", d64(x))],
        layers, d64(x), d64(dout), keep_hidden=True)
    e_x = e_src + e_dst + e_val
    # LeakyReLU's derivative jumps at z = 0: a hidden pre-activation within
    # fp32 rounding of 0 may take the other slope in fp32, which moves that
    # unit's dz by (1 - slope) |g| (g = dz / slope, the gradient at the
    # unit's output).  The kernel's z is a 20-term fp32 sum of exact fp32
    # products and inputs, so |z32 - z| <= 20 * 2^-24 * sum |W a| + |b|;
    # "near" takes 32 in place of 20.  The field gradients leave those
    # edges and the nodes they touch out; the hidden layer's weight and bias
    # gradients are held to 1e-5 of their largest element plus the sum of
    # those moves.
    a0, z0, dz0 = hidden[0]
    dst = graph.destination_index().long()
    w0, b0 = layers[0][0], layers[0][1]
    near = z0.abs() <= 32 * 2.0 ** -24 * (a0.abs() @ w0.abs().T + b0.abs())
    kink = near.any(1)
    touched = torch.zeros(N, dtype=torch.bool, device=DEV)
    touched[col.long()[kink]] = True
    touched[dst[kink]] = True
    print(f"  kink (edge, unit) pairs {int(near.sum())}, edges {int(kink.sum())}, "
          f"nodes they touch {int(touched.sum())}", flush=True)
    move = torch.where(near, 0.8 * (dz0 / torch.where(z0 > 0, 1.0, 0.2)).abs(),
                       torch.zeros_like(dz0))
    allow_w = move.T @ a0.abs()
    allow_b = move.sum(0)
    x_ok, e_ok = ~touched, ~kink
    checks = [("out", out, e_out, 1e-5), ("dx", x.grad[x_ok], e_x[x_ok], 1e-5),
              ("ddisplacement", disp.grad[e_ok], e_disp[e_ok], 1e-5),
              ("dW1", net[2].weight.grad, e_layers[1][0], 1e-5)]
    for name, got, want, tol in checks:
        err = rel(got, want)
        print(f"  {name}: max-norm {err:.2e} (bound {tol:g}); {elementwise(got, want)}",
              flush=True)
        assert err <= tol, name
    for name, got, want, allow in (("dW0", net[0].weight.grad, e_layers[0][0], allow_w),
                                   ("db0", net[0].bias.grad, e_layers[0][1], allow_b)):
        diff = (got.double() - want).abs()
        bound = 1e-5 * want.abs().max() + allow
        print(f"  {name}: max-norm {rel(got, want):.2e}, largest kink allowance "
              f"{float(allow.max() / want.abs().max()):.2e} of max; "
              f"worst diff / bound {float((diff / bound).max()):.3f}", flush=True)
        assert bool((diff <= bound).all()), name
    # The last bias shifts every score of a row alike: its exact gradient is
    # 0, so it is held to the scale of the last weight's gradient.
    db1 = net[2].bias.grad.double()
    assert float(db1.abs().max()) <= 1e-4 * float(e_layers[1][0].abs().max())

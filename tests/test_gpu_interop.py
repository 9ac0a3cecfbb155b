"""GPU checks of the Torch integration of the HIP path: the torch.library
registration (reference python/tiga/interop/torch/library.py:23-208) on ROCm
tensors, and HIP graph capture of a fused forward + backward.

Both must reproduce the direct HIP call bit for bit: they run the same
deterministic kernels on the same inputs.
"""

import numpy as np
import pytest
import torch

import tiga as tg

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


class GAT(tg.MessagePassing):
    """GAT additive attention as in the reference example
    (examples/gat_edge_attention.py), written with explicit vectors."""

    reducer = tg.online_softmax()

    def __init__(self, a_src, a_dst):
        super().__init__()
        self.a_src = a_src
        self.a_dst = a_dst

    def edge(self, src, dst, edge):
        score = torch.nn.functional.leaky_relu(
            (src.h * self.a_src).sum(-1) + (dst.h * self.a_dst).sum(-1), 0.2)
        return self.reducer(score, src.h)


def poisson_graph(n, mean, seed):
    rng = np.random.default_rng(seed)
    deg = rng.poisson(mean, n) + 1
    row_ptr = np.concatenate([[0], np.cumsum(deg)])
    col = np.concatenate([np.sort(np.append(rng.integers(0, n, d - 1), i))
                          for i, d in enumerate(deg)])
    return (torch.as_tensor(row_ptr, device=DEV), torch.as_tensor(col, device=DEV))


@pytest.fixture(autouse=True)
def strict():
    tg.config.strict = True
    yield
    tg.config.strict = False


def test_registered_op_runs_hip_path_and_matches_direct_call():
    print("torch.library GAT N=3000", flush=True)
    n, H, D = 3000, 4, 32
    row_ptr, col = poisson_graph(n, 8, 1)
    graph = tg.Graph.from_csr(row_ptr, col, num_src=n)
    g = torch.Generator(device=DEV).manual_seed(2)
    h = torch.randn(n, H, D, device=DEV, generator=g).requires_grad_(True)
    a_s = torch.randn(H, D, device=DEV, generator=g) * 0.1
    a_d = torch.randn(H, D, device=DEV, generator=g) * 0.1
    kernel = GAT(a_s, a_d)
    direct = kernel(graph=graph, src={"h": h}, dst={"h": h})
    assert kernel.last_variant.backend == "hip"
    dout = torch.randn_like(direct)
    (dh_direct,) = torch.autograd.grad(direct, (h,), dout)

    op = tg.interop.torch.register_message_passing(kernel, graph=graph, src={"h": h},
                                                   dst={"h": h}, name="gat_hip_test")
    assert op.qualified_name == "tiga::gat_hip_test"
    # The fields are operands in (src, dst, edge) order: h is passed twice.
    out = op(src={"h": h}, dst={"h": h})
    assert torch.equal(out, direct)
    (dh,) = torch.autograd.grad(out, (h,), dout)
    assert torch.equal(dh, dh_direct)

    # opcheck clones every operand separately, so dst.h is no longer src.h and
    # the GAT kernel (which needs one shared h) does not apply: the clones run
    # on the eager evaluator.  opcheck checks the registration (schema, fake
    # kernel, autograd formula, AOT); the HIP path is checked above.
    tg.config.strict = False
    checked = op.opcheck(h.detach(), h.detach())
    tg.config.strict = True
    assert all(result == "SUCCESS" for result in checked.values()), checked

    compiled = torch.compile(lambda x: op(src={"h": x}, dst={"h": x}), fullgraph=True)
    hc = h.detach().clone().requires_grad_(True)
    out_c = compiled(hc)
    (dh_c,) = torch.autograd.grad(out_c, (hc,), dout)
    assert torch.equal(out_c, direct)
    assert torch.equal(dh_c, dh_direct)


def test_hip_graph_capture_of_fused_forward_and_backward():
    """Capture GAT forward + backward in one HIP graph after a warm-up call
    built the per-graph plans; replay it several times with eager work and
    synchronisations in between, and compare every replay with the eager
    result."""
    print("hip graph capture GAT N=5000", flush=True)
    n, H, D = 5000, 8, 32
    row_ptr, col = poisson_graph(n, 12, 3)
    graph = tg.Graph.from_csr(row_ptr, col, num_src=n)
    g = torch.Generator(device=DEV).manual_seed(4)
    a_s = torch.randn(H, D, device=DEV, generator=g) * 0.1
    a_d = torch.randn(H, D, device=DEV, generator=g) * 0.1
    kernel = GAT(a_s, a_d)
    static_h = torch.randn(n, H, D, device=DEV, generator=g).requires_grad_(True)
    static_dout = torch.randn(n, H, D, device=DEV, generator=g)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):   # builds row plans and the transposed CSR (host syncs)
            static_h.grad = None
            kernel(graph=graph, src={"h": static_h}, dst={"h": static_h}).backward(static_dout)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph_exec = torch.cuda.CUDAGraph()
    static_h.grad = None
    with torch.cuda.graph(graph_exec):
        static_out = kernel(graph=graph, src={"h": static_h}, dst={"h": static_h})
        static_out.backward(static_dout)

    for replay in range(4):
        fresh = torch.randn(n, H, D, device=DEV, generator=g)
        with torch.no_grad():
            static_h.copy_(fresh)
        graph_exec.replay()
        torch.cuda.synchronize()
        got_out, got_dh = static_out.clone(), static_h.grad.clone()
        # eager reference on the same inputs, between replays
        h = fresh.clone().requires_grad_(True)
        out = kernel(graph=graph, src={"h": h}, dst={"h": h})
        out.backward(static_dout)
        torch.cuda.synchronize()
        assert torch.equal(got_out, out.detach()), f"replay {replay}: output differs"
        assert torch.equal(got_dh, h.grad), f"replay {replay}: gradient differs"


class DotBias(tg.MessagePassing):
    reducer = tg.online_softmax()

    def edge(self, src, dst, edge, scale):
        return self.reducer((src.k * dst.q).sum(dim=-1) * scale + edge.bias, src.v)


def test_hip_graph_capture_of_dot_attention_with_kept_score_gradients():
    """Capture dot-product attention forward + backward (whose source pass
    keeps each edge's score gradient for the destination pass) on an R-MAT
    graph with hub rows split on both sides; every replay, with eager work in
    between, equals the eager step bit for bit."""
    from graphs import rmat_csr

    print("hip graph capture dot R-MAT scale 11", flush=True)
    rp, cl = rmat_csr(9, 11)
    n, E, H, D = rp.size - 1, cl.size, 4, 64
    graph = tg.Graph.from_csr(torch.as_tensor(rp, device=DEV), torch.as_tensor(cl, device=DEV),
                              num_src=n)
    g = torch.Generator(device=DEV).manual_seed(5)
    mk = lambda *shape: torch.randn(*shape, device=DEV, generator=g)
    q, k, v = (mk(n, H, D).to(torch.bfloat16).requires_grad_(True) for _ in range(3))
    bias = mk(E, H).requires_grad_(True)
    dout = mk(n, H, D).to(torch.bfloat16)
    kernel = DotBias()
    leaves = (q, k, v, bias)

    def step(tensors):
        out = kernel(graph=graph, src={"k": tensors[1], "v": tensors[2]}, dst={"q": tensors[0]},
                     edge={"bias": tensors[3]}, scale=0.125)
        out.backward(dout)
        return out

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):   # builds row plans and the transposed CSR (host syncs)
            for t in leaves:
                t.grad = None
            step(leaves)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert kernel.last_variant.backend == "hip"

    graph_exec = torch.cuda.CUDAGraph()
    for t in leaves:
        t.grad = None
    with torch.cuda.graph(graph_exec):
        static_out = step(leaves)

    for replay in range(4):
        fresh = [mk(*t.shape).to(t.dtype) for t in leaves]
        with torch.no_grad():
            for t, f in zip(leaves, fresh):
                t.copy_(f)
        graph_exec.replay()
        torch.cuda.synchronize()
        got = [static_out.clone()] + [t.grad.clone() for t in leaves]
        eager = [f.clone().requires_grad_(True) for f in fresh]
        out = step(eager)
        torch.cuda.synchronize()
        want = [out.detach()] + [t.grad for t in eager]
        for name, a, b in zip(("out", "dq", "dk", "dv", "dbias"), got, want):
            assert torch.equal(a, b), f"replay {replay}: {name} differs"

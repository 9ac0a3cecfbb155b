"""GPU parity of the MFMA attention tiles on dense relations (Graph.dense,
Graph.triangular), non-causal varlen relations, fp16 and bf16, head_dim 64
and 128, and the block-pruned forward, against the fp64 oracle.

Tolerances: max|gpu - oracle| <= tol * max|oracle| per tensor, tol = 5e-3 for
fp16 inputs (11-bit softmax weights), 2e-2 for bf16 (the north star's bf16
bound).  The reference's own example checks (tests/python/
test_attention_examples.py:25-90) use rtol = atol = 3e-3..4e-3 against SDPA
for fp16.
"""

import numpy as np
import pytest
import torch

import tiga as tg
from oracle import ref

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
TOL = {torch.float16: 5e-3, torch.bfloat16: 2e-2}


def rel_err(actual, expected):
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    return float(np.abs(a - e).max() / max(np.abs(e).max(), 1e-30))


def f64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


class DotAttention(tg.MessagePassing):
    """The reference examples' kernel (examples/full_attention.py:16-22)."""

    reducer = tg.online_softmax()

    def edge(self, src, dst, edge, scale):
        score = (src.key * dst.query).sum(dim=-1) * scale
        return self.reducer(score, src.value)


class TilePrunedAttention(tg.MessagePassing):
    """examples/tile_pruned_attention.py:16-26."""

    def __init__(self, threshold):
        super().__init__()
        self.reducer = tg.online_softmax(block_prune_threshold=threshold)

    def edge(self, src, dst, edge, scale):
        score = (src.key * dst.query).sum(dim=-1) * scale
        return self.reducer(score, src.value)


def lane_major(heads, nodes, width, dtype, gen):
    """The reference examples' layout: (H, N, D) storage viewed as (N, H, D)."""
    return torch.randn(heads, nodes, width, device=DEV, dtype=dtype, generator=gen).permute(1, 0, 2)


@pytest.fixture(autouse=True)
def strict():
    tg.config.strict = True
    yield
    tg.config.strict = False


def test_full_attention_example():
    """examples/full_attention.py: dense 1024 x 1024, H=4, D=64, fp16."""
    print("dense fp16 1024x4x64", flush=True)
    g = torch.Generator(device=DEV).manual_seed(0)
    nodes, heads, width = 1024, 4, 64
    query, key, value = (lane_major(heads, nodes, width, torch.float16, g) for _ in range(3))
    program = DotAttention()
    output = program(graph=tg.Graph.dense(nodes, device="cuda"), src={"key": key, "value": value},
                     dst={"query": query}, scale=width ** -0.5)
    assert program.last_variant.backend == "hip"
    assert output.shape == (nodes, heads, width) and output.dtype == torch.float16
    expect, _ = ref.block_attention_fwd([0, nodes], [0, nodes], f64(query), f64(key),
                                        f64(value), width ** -0.5, False)
    assert rel_err(f64(output), expect) <= TOL[torch.float16]


def test_causal_dense_relation_example():
    """examples/causal_dense_relation.py: triangular 256, H=2, D=64, fp16."""
    print("triangular fp16 256x2x64", flush=True)
    g = torch.Generator(device=DEV).manual_seed(7)
    nodes, heads, width = 256, 2, 64
    query, key, value = (lane_major(heads, nodes, width, torch.float16, g) for _ in range(3))
    graph = tg.Graph.triangular(nodes, device="cuda")
    assert graph.schema.origin == "lower_triangular" and graph.num_edges == nodes * (nodes + 1) // 2
    output = DotAttention()(graph=graph, src={"key": key, "value": value}, dst={"query": query},
                            scale=width ** -0.5)
    expect, _ = ref.block_attention_fwd([0, nodes], [0, nodes], f64(query), f64(key),
                                        f64(value), width ** -0.5, True)
    assert rel_err(f64(output), expect) <= TOL[torch.float16]


@pytest.mark.parametrize("dtype,D,n_dst,n_src,causal,layout", [
    (torch.bfloat16, 128, 300, 700, False, "lane_major"),
    (torch.float16, 64, 513, 130, False, "contiguous"),
    (torch.bfloat16, 64, 333, 333, True, "contiguous"),
    (torch.float16, 128, 200, 200, True, "lane_major"),
    (torch.bfloat16, 32, 300, 450, False, "lane_major"),
    (torch.float16, 32, 333, 333, True, "contiguous"),
])
def test_dense_fwd_bwd(dtype, D, n_dst, n_src, causal, layout):
    print(f"dense {dtype} D={D} {n_dst}x{n_src} causal={causal} {layout}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(n_dst + n_src + D)
    H = 3

    def make(n):
        if layout == "lane_major":
            t = torch.randn(H, n, D, device=DEV, generator=g).to(dtype).permute(1, 0, 2)
        else:
            t = torch.randn(n, H, D, device=DEV, generator=g).to(dtype)
        return t.requires_grad_(True)

    q, k, v = make(n_dst), make(n_src), make(n_src)
    graph = (tg.Graph.triangular(n_dst, device=DEV) if causal
             else tg.Graph.dense(n_src, n_dst, device=DEV))
    kernel = DotAttention()
    out = kernel(graph=graph, src={"key": k, "value": v}, dst={"query": q}, scale=D ** -0.5)
    assert kernel.last_variant.backend == "hip"
    dout = torch.randn(n_dst, H, D, device=DEV, generator=g).to(dtype)
    out.backward(dout)
    cu_q, cu_k = [0, n_dst], [0, n_src]
    e_out, _ = ref.block_attention_fwd(cu_q, cu_k, f64(q), f64(k), f64(v), D ** -0.5, causal)
    e_grads = ref.block_attention_bwd(cu_q, cu_k, f64(q), f64(k), f64(v), D ** -0.5, causal,
                                      f64(dout))
    tol = TOL[dtype]
    assert rel_err(f64(out), e_out) <= tol
    for got, exp in zip((q.grad, k.grad, v.grad), e_grads):
        assert rel_err(f64(got), exp) <= tol


@pytest.mark.parametrize("dtype,D", [(torch.float16, 128), (torch.bfloat16, 64),
                                     (torch.bfloat16, 32)])
def test_noncausal_varlen_fwd_bwd(dtype, D):
    print(f"varlen non-causal {dtype} D={D}", flush=True)
    lengths = [1, 130, 0, 64, 257, 5]
    cu = np.concatenate([[0], np.cumsum(lengths)])
    T, H = int(cu[-1]), 2
    g = torch.Generator(device=DEV).manual_seed(D)
    q, k, v = (torch.randn(T, H, D, device=DEV, generator=g).to(dtype).requires_grad_(True)
               for _ in range(3))
    graph = tg.Graph.cu_seqlens(torch.as_tensor(cu, device=DEV), causal=False)
    out = DotAttention()(graph=graph, src={"key": k, "value": v}, dst={"query": q}, scale=0.1)
    dout = torch.randn(T, H, D, device=DEV, generator=g).to(dtype)
    out.backward(dout)
    e_out, _ = ref.block_attention_fwd(cu, cu, f64(q), f64(k), f64(v), 0.1, False)
    e_grads = ref.block_attention_bwd(cu, cu, f64(q), f64(k), f64(v), 0.1, False, f64(dout))
    tol = TOL[dtype]
    assert rel_err(f64(out), e_out) <= tol
    for got, exp in zip((q.grad, k.grad, v.grad), e_grads):
        assert rel_err(f64(got), exp) <= tol


def test_tile_pruned_example_is_finite_and_matches_oracle():
    """examples/tile_pruned_attention.py (threshold = width / nodes).  Random
    scores never trail a block's running max by 4 log2 units, so every tile
    is admitted: the output is exact attention and finite (the reference's
    own check, test_attention_examples.py:75-90)."""
    print("pruned example fp16 1024x4x64", flush=True)
    g = torch.Generator(device=DEV).manual_seed(0)
    nodes, heads, width = 1024, 4, 64
    query, key, value = (lane_major(heads, nodes, width, torch.float16, g) for _ in range(3))
    program = TilePrunedAttention(width / nodes)
    output = program(graph=tg.Graph.dense(nodes, device="cuda"),
                     src={"key": key, "value": value}, dst={"query": query},
                     scale=width ** -0.5)
    assert torch.isfinite(output).all()
    assert output.shape == (nodes, heads, width)
    cu = [0, nodes]
    expect, _ = ref.block_pruned_attention_fwd(cu, cu, f64(query), f64(key), f64(value),
                                               width ** -0.5, width / nodes, False)
    assert rel_err(f64(output), expect) <= TOL[torch.float16]


@pytest.mark.parametrize("causal", [False, True])
def test_block_pruning_skips_the_known_tile(causal):
    """Admission is decided per 128-query block (Translate.cpp:1793-1815):
    queries 0-63 are u and 64-127 are -u; keys 0-63 are 16u and 64-127 are
    -4u.  Scores: rows < 64 see +8 then -2, rows >= 64 see -8 then +2.  The
    block's running max after tile 0 is 8, tile 1's max is 2: a log2 gap of
    8.66 > 5, so with threshold 2^-5 tile 1 is skipped for the whole block,
    although exact softmax puts nearly all of rows 64-127's weight on it."""
    print(f"pruned known tile causal={causal}", flush=True)
    n, H, D = 128, 1, 64
    u = torch.full((D,), 0.25)
    sign_q = torch.tensor([1.0, -1.0]).repeat_interleave(64)
    q = (sign_q[:, None] * u).reshape(n, H, D).to(torch.float16).to(DEV)
    k = torch.cat([16.0 * u.expand(64, D), -4.0 * u.expand(64, D)]).reshape(n, H, D)
    k = k.to(torch.float16).to(DEV)
    g = torch.Generator(device=DEV).manual_seed(3)
    v = torch.randn(n, H, D, device=DEV, generator=g).to(torch.float16)
    graph = tg.Graph.triangular(n, device=DEV) if causal else tg.Graph.dense(n, device=DEV)
    with torch.no_grad():
        out = TilePrunedAttention(2.0 ** -5)(graph=graph, src={"key": k, "value": v},
                                             dst={"query": q}, scale=D ** -0.5)
    got = f64(out)
    expect, _ = ref.block_pruned_attention_fwd([0, n], [0, n], f64(q), f64(k), f64(v),
                                               D ** -0.5, 2.0 ** -5, causal)
    assert rel_err(got, expect) <= TOL[torch.float16]
    vv = f64(v)[:, 0]
    for i in (0, 10, 63, 64, 100, 127):
        keys = np.arange(min(i + 1, 64) if causal else 64)   # tile 0 only, equal scores
        np.testing.assert_allclose(got[i, 0], vv[keys].mean(0), rtol=0, atol=5e-3)
    exact, _ = ref.block_attention_fwd([0, n], [0, n], f64(q), f64(k), f64(v), D ** -0.5, causal)
    assert np.abs(exact[64:] - expect[64:]).max() > 0.1     # pruning changed those rows


def test_pruning_fails_closed():
    g = torch.Generator(device=DEV).manual_seed(1)
    n, H, D = 128, 2, 64
    q, k, v = (torch.randn(n, H, D, device=DEV, generator=g).to(torch.float16)
               for _ in range(3))
    prog = TilePrunedAttention(0.5)
    with pytest.raises(NotImplementedError, match="forward-only"):
        prog(graph=tg.Graph.dense(n, device=DEV),
             src={"key": k.requires_grad_(True), "value": v}, dst={"query": q}, scale=0.1)
    rp = torch.arange(n + 1, device=DEV) * 4
    col = torch.randint(0, n, (4 * n,), device=DEV, generator=g)
    with pytest.raises(NotImplementedError, match="dense relations only"):
        with torch.no_grad():
            prog(graph=tg.Graph.from_csr(rp, col, num_src=n), src={"key": k, "value": v},
                 dst={"query": q}, scale=0.1)
    with pytest.raises(NotImplementedError, match="dense attention tile"):
        with torch.no_grad():   # head_dim 48 has no tile
            prog(graph=tg.Graph.dense(n, device=DEV), src={"key": k[..., :48], "value": v[..., :48]},
                 dst={"query": q[..., :48]}, scale=0.1)


def test_dense_uncovered_edge_function_runs_eager_on_materialized_relation():
    """An edge function no tile covers materializes the dense CSR (device
    builder) and runs the eager evaluator, as the reference's generic path."""
    tg.config.strict = False

    class ScaledValue(tg.MessagePassing):
        reducer = tg.online_softmax()

        def edge(self, src, dst, edge):
            return self.reducer((src.key * dst.query).sum(dim=-1).tanh(), src.value)

    g = torch.Generator(device=DEV).manual_seed(2)
    q = torch.randn(9, 2, 4, device=DEV, generator=g)
    k, v = (torch.randn(5, 2, 4, device=DEV, generator=g) for _ in range(2))
    graph = tg.Graph.dense(5, 9, device=DEV)
    prog = ScaledValue()
    out = prog(graph=graph, src={"key": k, "value": v}, dst={"query": q})
    assert prog.last_variant.backend == "torch-eager"
    s = np.tanh(np.einsum("ihd,jhd->hij", f64(q), f64(k)))
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    np.testing.assert_allclose(f64(out), np.einsum("hij,jhd->ihd", p, f64(v)), rtol=1e-5,
                               atol=1e-6)


def torch_block_attention(q, k, v, scale, causal):
    """fp32 Torch attention over one block ([n, H, D] in, [n, H, D] out)."""
    qf, kf, vf = (t.detach().float().permute(1, 0, 2).contiguous() for t in (q, k, v))
    s = torch.matmul(qf, kf.transpose(1, 2).contiguous()) * scale
    if causal:
        n = s.shape[-1]
        s.masked_fill_(torch.ones(n, n, dtype=torch.bool, device=DEV).triu(1), float("-inf"))
    return torch.matmul(torch.softmax(s, dim=-1), vf).permute(1, 0, 2)


@pytest.mark.parametrize("n,H,D,causal,dtype", [
    (4096, 16, 64, True, torch.float16),     # the reference's causal dense case: 2 chunks
    (8192, 2, 128, True, torch.bfloat16),    # up to 8 chunks per tile
    (4096, 4, 64, False, torch.bfloat16),    # few, equal tiles: 4 chunks each
    ((4096, 3000, 100), 4, 128, True, torch.float16),   # causal cu_seqlens, 3 blocks
    (4096, 4, 32, True, torch.bfloat16),     # head dim 32
])
def test_split_key_ranges_match_whole_tiles(n, H, D, causal, dtype):
    """Relations with too few query tiles to fill the GPU run the longest key
    ranges in chunks (tgx_attn_fwd_split) and merge them: the output matches
    fp32 attention, and the forward and the gradients match the whole-tile
    forward's up to the order of the softmax sums."""
    print(f"split forward n={n} H={H} D={D} causal={causal} {dtype}", flush=True)
    lengths = n if isinstance(n, tuple) else None
    n = sum(lengths) if lengths else n
    g = torch.Generator(device=DEV).manual_seed(n + H + D)
    base = [torch.randn(n, H, D, device=DEV, generator=g).to(dtype) for _ in range(4)]
    results = []
    for split in (True, False):
        if lengths:
            cu = torch.tensor([0, *np.cumsum(lengths)], dtype=torch.int64, device=DEV)
            graph = tg.Graph.cu_seqlens(cu, causal=True)
        else:
            graph = (tg.Graph.triangular(n, device=DEV) if causal
                     else tg.Graph.dense(n, device=DEV))
        if split:
            plan = graph._attn_fwd_split(H)
            assert plan is not None and plan[3] > 0
        else:
            graph._native_cache[("attn-split", H)] = None   # whole tiles only
        q, k, v = (t.clone().requires_grad_(True) for t in base[:3])
        kernel = DotAttention()
        out = kernel(graph=graph, src={"key": k, "value": v}, dst={"query": q},
                     scale=D ** -0.5)
        assert kernel.last_variant.backend == "hip"
        out.backward(base[3])
        results.append((out.detach().float(), q.grad.float(), k.grad.float(), v.grad.float()))
    tol = TOL[dtype]
    starts = np.cumsum([0, *lengths]) if lengths else [0, n]
    for s0, s1 in zip(starts[:-1], starts[1:]):
        expect = torch_block_attention(base[0][s0:s1], base[1][s0:s1], base[2][s0:s1],
                                       D ** -0.5, causal)
        got = results[0][0][s0:s1]
        assert float((got - expect).abs().max() / expect.abs().max()) <= tol
    for a, b in zip(results[0], results[1]):
        assert float((a - b).abs().max() / b.abs().max()) <= tol

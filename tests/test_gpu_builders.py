"""GPU parity of the device graph builders (Graph.from_coo, Graph.transpose,
Graph.destination_index, the materialized Graph.cu_seqlens CSR) against the
CPU oracle.  Integer outputs: bit-exact, including the output dtypes the
reference constructors produce (row_ptr in dst's dtype, col_idx in src's).
"""

import numpy as np
import pytest
import torch

import tiga as tg
from oracle import ref

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def _eq(t, a):
    return np.array_equal(t.cpu().numpy().astype(np.int64), np.asarray(a, dtype=np.int64))


@pytest.mark.parametrize("src_dtype,dst_dtype", [(torch.int32, torch.int32),
                                                 (torch.int64, torch.int64),
                                                 (torch.int32, torch.int64),
                                                 (torch.int64, torch.int32)])
@pytest.mark.parametrize("n_src,n_dst,E", [(7, 5, 0), (30, 20, 200), (1000, 70000, 300000),
                                           (5000, 3_000_000, 1_000_000)])
def test_from_coo_matches_oracle(src_dtype, dst_dtype, n_src, n_dst, E):
    print(f"from_coo {src_dtype} {dst_dtype} n_src={n_src} n_dst={n_dst} E={E}", flush=True)
    rng = np.random.default_rng(n_dst + E)
    src = rng.integers(0, n_src, E)
    dst = rng.integers(0, n_dst, E)
    dst[: E // 4] = dst[0] if E else 0          # a hub row with many duplicates
    g = tg.Graph.from_coo(torch.as_tensor(src, dtype=src_dtype, device=DEV),
                          torch.as_tensor(dst, dtype=dst_dtype, device=DEV),
                          num_src=n_src, num_dst=n_dst)
    rp, col = g.resolve_csr()
    erp, ecol, _ = ref.from_coo(src, dst, num_src=n_src, num_dst=n_dst)
    assert rp.dtype == dst_dtype and col.dtype == src_dtype
    assert _eq(rp, erp) and _eq(col, ecol)
    assert g.schema.num_src == n_src and g.schema.num_dst == n_dst


def test_from_coo_infers_sizes_and_rejects_out_of_range():
    src = torch.tensor([2, 0, 1, 2], device=DEV)
    dst = torch.tensor([1, 1, 0, 3], device=DEV)
    g = tg.Graph.from_coo(src, dst)
    erp, ecol, ns = ref.from_coo(src.cpu().numpy(), dst.cpu().numpy())
    rp, col = g.resolve_csr()
    assert _eq(rp, erp) and _eq(col, ecol) and g.schema.num_src == ns
    with pytest.raises(ValueError, match="out-of-range destination"):
        tg.Graph.from_coo(src, dst, num_dst=3)


@pytest.mark.parametrize("dtype", [torch.int32, torch.int64])
def test_transpose_and_destination_index_match_oracle(dtype):
    print(f"transpose {dtype}", flush=True)
    rng = np.random.default_rng(11)
    n_src, n_dst, E = 40_000, 25_000, 400_000
    src = rng.integers(0, n_src, E)
    dst = np.sort(rng.integers(0, n_dst, E))
    erp, ecol, _ = ref.from_coo(src, dst, num_src=n_src, num_dst=n_dst)
    g = tg.Graph.from_csr(torch.as_tensor(erp, dtype=dtype, device=DEV),
                          torch.as_tensor(ecol, dtype=dtype, device=DEV), num_src=n_src)
    d = g.destination_index()
    assert d.dtype == torch.int64 and _eq(d, ref.destination_index(erp))
    t = g.transpose()
    trp, tcol, _ = ref.transpose(erp, ecol, n_src)
    rp, col = t.resolve_csr()
    assert rp.dtype == dtype and col.dtype == dtype
    assert _eq(rp, trp) and _eq(col, tcol)
    assert t.schema.num_src == n_dst and t.schema.num_dst == n_src
    # transposing twice sorts every row's sources (stable order by source)
    rp2, col2 = t.transpose().resolve_csr()
    erp2, ecol2, _ = ref.transpose(trp, tcol, n_dst)
    assert _eq(rp2, erp) and _eq(rp2, erp2) and _eq(col2, ecol2)
    order = np.lexsort((ecol, ref.destination_index(erp)))
    assert _eq(col2, ecol[order])


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("dtype", [torch.int32, torch.int64])
def test_varlen_csr_matches_oracle(causal, dtype):
    print(f"varlen csr causal={causal} {dtype}", flush=True)
    rng = np.random.default_rng(5 + causal)
    lengths = rng.integers(0, 300, 24)
    lengths[[0, 5, 6, 23]] = 0                    # empty sequences, leading and trailing
    lengths[9] = 1
    cu = np.concatenate([[0], np.cumsum(lengths)])
    g = tg.Graph.cu_seqlens(torch.as_tensor(cu, dtype=dtype, device=DEV), causal=causal)
    rp, col = g.resolve_csr()
    erp, ecol = ref.cu_seqlens_csr(cu, causal=causal)
    assert rp.dtype == dtype and col.dtype == dtype
    assert _eq(rp, erp) and _eq(col, ecol)
    assert g.num_edges == ecol.size


def test_varlen_csr_single_and_empty():
    g = tg.Graph.triangular(1000, device=DEV)
    rp, col = g.resolve_csr()
    erp, ecol = ref.cu_seqlens_csr([0, 1000])
    assert _eq(rp, erp) and _eq(col, ecol)
    g0 = tg.Graph.cu_seqlens(torch.zeros(3, dtype=torch.int64, device=DEV))
    rp0, col0 = g0.resolve_csr()
    assert _eq(rp0, [0]) and col0.numel() == 0


def test_builders_do_not_use_torch_sorting(monkeypatch):
    """On the GPU the constructors run this library's kernels: the Torch ops
    the reference builds them from are never reached."""
    def refuse(*args, **kwargs):
        raise AssertionError("Torch graph-construction op called on the GPU path")

    src = torch.randint(0, 100, (5000,), device=DEV)
    dst = torch.randint(0, 100, (5000,), device=DEV)
    for name in ("argsort", "bincount", "repeat_interleave"):
        monkeypatch.setattr(torch, name, refuse)
    g = tg.Graph.from_coo(src, dst, num_src=100, num_dst=100)
    g.destination_index()
    g.transpose()
    tg.Graph.cu_seqlens(torch.tensor([0, 7, 20], device=DEV), causal=False).resolve_csr()

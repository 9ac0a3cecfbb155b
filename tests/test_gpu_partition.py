"""The reference's degree buckets on the device partition.

The reference planner's bucket bounds (tgx_plan_reference_buckets, pinned by
the lit vectors in tests/test_host.py; PlanDegreeBuckets.cpp:86-143) are fed
to the device partition tgx_plan_degree_bins, and the result is compared bit
for bit with ref.degree_bins (ascending row ids inside each bucket; the
reference's atomic worklist scatter fixes only the membership,
Translate.cpp:4043-4187) and with the planner's own rows-per-bucket counts.

Graphs: the lit vectors' degree histograms scaled up with shuffled rows,
power-law rows with hubs, and R-MAT scale 12.
"""

import ctypes

import numpy as np
import pytest
import torch

import tiga as tg
from tiga import _native
from tiga.graph import reference_plan
from oracle import ref

from graphs import rmat_csr, skewed_csr

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def _from_histogram(hist: dict, scale: int, seed: int):
    rng = np.random.default_rng(seed)
    deg = np.concatenate([np.full(count * scale, d, dtype=np.int64)
                          for d, count in hist.items()])
    rng.shuffle(deg)
    rp = np.zeros(deg.size + 1, dtype=np.int64)
    np.cumsum(deg, out=rp[1:])
    return rp


def _device_bins(rp: np.ndarray, bounds, idx):
    n = rp.size - 1
    row_ptr = torch.as_tensor(rp, device=DEV).to(idx)
    ws_bytes = ctypes.c_size_t()
    _native.call("tgx_plan_degree_bins_workspace", n, len(bounds), ctypes.byref(ws_bytes))
    ws = torch.empty(max(ws_bytes.value, 1), dtype=torch.uint8, device=DEV)
    rows = torch.empty(max(n, 1), dtype=torch.int32, device=DEV)
    ub = (ctypes.c_int64 * len(bounds))(*bounds)
    offsets = (ctypes.c_int64 * (len(bounds) + 1))()
    _native.call("tgx_plan_degree_bins", row_ptr.data_ptr(), _native.idx_bits(row_ptr), n, ub,
                 len(bounds), rows.data_ptr(), offsets, ws.data_ptr(), ws_bytes.value,
                 _native.stream_of(row_ptr))
    return rows[:n].cpu().numpy(), list(offsets)


CASES = {
    # tests/mlir/power-law-cdf-split.mlir, plan-split-rows.mlir (histogram
    # {8: 120, 64: 7, 256: 1}), tail-split-to-bundle.mlir ({8: 384, 32: 102,
    # 64: 26}) and kernel-load-balance-analysis.mlir's padding-poor shape.
    "lit-power-law-x40": lambda: _from_histogram({8: 120, 64: 7, 256: 1}, 40, 1),
    "lit-tail-split-x20": lambda: _from_histogram({8: 384, 32: 102, 64: 26}, 20, 2),
    "lit-padding-poor-x30": lambda: _from_histogram({0: 64, 1: 32, 64: 32}, 30, 3),
    "power-law-hubs": lambda: skewed_csr(5, 20000, 20000, mean_deg=5,
                                         hubs=(3000, 800, 200, 65, 64))[0],
    "rmat-scale-12": lambda: rmat_csr(6, 12)[0],
}


@pytest.mark.parametrize("name", sorted(CASES))
@pytest.mark.parametrize("has_node", [False, True])
@pytest.mark.parametrize("idx", [torch.int32, torch.int64])
def test_reference_buckets_on_the_device_partition(name, has_node, idx):
    rp = CASES[name]()
    deg = np.diff(rp)
    hist = np.bincount(deg, minlength=deg.max() + 1).tolist() if deg.max() <= 4096 else None
    plan = reference_plan(deg.size, int(deg.max()), int(deg.sum()), hist, has_node)
    print(f"{name} node={has_node} {idx}: {plan['plan']} bounds {plan['bounds']}", flush=True)
    if not plan["bounds"]:
        pytest.skip(f"the reference plans no buckets here ({plan['plan']})")
    bounds = plan["bounds"]
    assert len(bounds) <= 8
    rows, offsets = _device_bins(rp, bounds, idx)
    e_rows, e_off = ref.degree_bins(rp, bounds)
    assert offsets == e_off.tolist()
    assert rows.tolist() == e_rows.tolist()
    counts = np.diff(offsets).tolist()
    # The last bucket also takes every degree above its bound (none here:
    # the planner's last bound is the maximum degree).
    assert counts == plan["rows_in_bucket"]
    # Membership by the reference's rule: lower < degree <= upper.
    lower = -1
    for b, upper in enumerate(bounds):
        members = rows[offsets[b]:offsets[b + 1]]
        assert ((deg[members] > lower) & (deg[members] <= upper)).all()
        lower = upper

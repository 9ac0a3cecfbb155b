"""tgx_dot_attn_fwd_noalloc: the dot-product forward with its split-row
partials in the library's static device scratch instead of a caller
buffer.  Checked through the C ABI against tgx_dot_attn_fwd on the same
plan and inputs (the same kernels, so bit-identical), on two calls in a
row, the second smaller, and on two streams; and its size limit is rejected
before any launch."""

import ctypes

import numpy as np
import pytest
import torch

from tiga import _native
from tiga.graph import build_row_plan

from graphs import skewed_csr


def _case(seed, n, hubs, H, D, idx):
    dev = torch.device("cuda")
    rp, col = skewed_csr(seed, n, n, mean_deg=6, hubs=hubs)
    row_ptr = torch.tensor(rp, device=dev, dtype=idx)
    col_t = torch.tensor(col, device=dev, dtype=idx)
    g = torch.Generator(device=dev).manual_seed(seed)
    q, k, v = (torch.randn(n, H, D, device=dev, generator=g).to(torch.bfloat16)
               for _ in range(3))
    bias = torch.randn(col.size, H, device=dev, generator=g)
    plan = build_row_plan(row_ptr, n)
    return row_ptr, col_t, plan, q, k, v, bias


def _forward(name, row_ptr, col, plan, q, k, v, bias, scale, partial=()):
    n, H, D = q.shape
    out = torch.empty_like(q)
    ml = torch.empty(n, H, 2, device=q.device)
    _native.call(name, row_ptr.data_ptr(), col.data_ptr(), _native.idx_bits(row_ptr), plan.ref,
                 q.data_ptr(), k.data_ptr(), v.data_ptr(), bias.data_ptr(), scale,
                 out.data_ptr(), ml.data_ptr(), n, n, H, D, 0, *partial,
                 _native.stream_of(q))
    return out, ml


@pytest.mark.gpu
def test_noalloc_forward_matches_the_caller_buffer_forward_twice():
    for seed, n, hubs, H, D, idx in ((0, 20000, (9000, 5000, 2600, 700), 4, 64, torch.int64),
                                     (1, 3000, (1500,), 2, 64, torch.int32)):
        print(f"noalloc seed={seed} n={n} hubs={hubs} H={H} D={D} {idx}", flush=True)
        row_ptr, col, plan, q, k, v, bias = _case(seed, n, hubs, H, D, idx)
        assert plan.plan.n_chunks > 0
        partial = torch.empty(plan.plan.n_chunks * (H * D + 2 * H), device=q.device)
        want = _forward("tgx_dot_attn_fwd", row_ptr, col, plan, q, k, v, bias, 0.125,
                        (partial.data_ptr(),))
        got = _forward("tgx_dot_attn_fwd_noalloc", row_ptr, col, plan, q, k, v, bias, 0.125)
        torch.cuda.synchronize()
        assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])


@pytest.mark.gpu
def test_noalloc_calls_on_two_streams_run_in_call_order():
    """Two uncaptured calls on different streams share the device's scratch:
    the second waits for the first (an event recorded after it), so both
    match the caller-buffer forward."""
    print("noalloc on two streams", flush=True)
    cases = [_case(0, 20000, (9000, 5000, 2600, 700), 4, 64, torch.int64),
             _case(1, 3000, (1500,), 2, 64, torch.int32)]
    want = []
    for row_ptr, col, plan, q, k, v, bias in cases:
        n, H, D = q.shape
        partial = torch.empty(plan.plan.n_chunks * (H * D + 2 * H), device=q.device)
        want.append(_forward("tgx_dot_attn_fwd", row_ptr, col, plan, q, k, v, bias, 0.125,
                             (partial.data_ptr(),)))
    torch.cuda.synchronize()
    got = []
    for case, stream in zip(cases, (torch.cuda.Stream(), torch.cuda.Stream())):
        with torch.cuda.stream(stream):
            got.append(_forward("tgx_dot_attn_fwd_noalloc", *case, 0.125))
    torch.cuda.synchronize()
    for (o, ml), (wo, wml) in zip(got, want):
        assert torch.equal(o, wo) and torch.equal(ml, wml)


def test_noalloc_forward_rejects_plans_beyond_its_scratch():
    # Checked on the host before any HIP call: no device is touched.
    H, D = 4, 64
    per_chunk = (H * D + 2 * H) * 4
    too_many = (64 << 20) // per_chunk + 1
    plan = _native.RowPlan(10, 0, 9, 1, too_many, 512, 512, 1, 1)
    with pytest.raises(RuntimeError, match="static scratch holds"):
        _native.call("tgx_dot_attn_fwd_noalloc", None, None, 64, ctypes.byref(plan), None,
                     None, None, None, 0.125, None, None, 10, 10, H, D, 0, None)

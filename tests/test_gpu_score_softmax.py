"""Online softmax over a raw score field on the HIP path:
reducer(role.score [* c], src.value) for a source-node, destination-node or
edge score field.

Checked against the reference's own known answer (scores about 1000, the
native-path test tests/python/test_message_passing_autograd.py:318-351,
restated in tests/golden/reference_vectors.json) and against the float64
oracle (ref.segment_softmax / segment_softmax_bwd, pinned by the same known
answer and finite differences) on graphs with hub rows and empty rows; fp32
outputs and gradients within 1e-5 relative.

Empty rows give 0, as the reference's Torch path does (test_reference.py:
416-444); its native tg.Tensor path gives 0/0 = NaN there
(message_passing/core.py:423-440), which this provider does not reproduce.
"""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

import tiga as tg
from oracle import ref

from graphs import skewed_csr

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
GOLD = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())


@pytest.fixture(autouse=True)
def _strict():
    tg.config.strict = True
    yield
    tg.config.strict = False


class OnlineAttention(tg.MessagePassing):
    """The reference's kernel of the known-answer test, unchanged."""

    reducer = tg.online_softmax()

    def edge(self, src, dst, edge):
        del dst, edge
        return self.reducer(src.score, src.value)


def rel(a, e):
    a, e = np.asarray(a, np.float64), np.asarray(e, np.float64)
    return float(np.abs(a - e).max() / max(np.abs(e).max(), 1e-30))


def test_reference_known_answer_at_large_scores():
    g = GOLD["online_softmax_large_scores"]
    graph = tg.Graph.from_csr(torch.tensor(g["row_ptr"], device=DEV),
                              torch.tensor(g["col_idx"], device=DEV), num_src=g["num_src"])
    score = torch.tensor(g["score"], device=DEV, requires_grad=True)
    value = torch.tensor(g["value"], device=DEV, requires_grad=True)
    k = OnlineAttention()
    out = k(graph=graph, src={"score": score, "value": value}, dst={})
    assert k.last_variant.backend == "hip" and k.last_variant.pattern == "score-softmax"
    dscore, dvalue = torch.autograd.grad(out.sum(), (score, value))
    tol = 0.5 * 10.0 ** -g["places"]
    np.testing.assert_allclose(out.detach().cpu().numpy(), g["out"], rtol=0, atol=tol)
    np.testing.assert_allclose(dscore.cpu().numpy(), g["dscore"], rtol=0, atol=tol)
    np.testing.assert_allclose(dvalue.cpu().numpy(), g["dvalue"], rtol=0, atol=tol)


def _expected(rp, col, table, role, scale, value, dout):
    """fp64 oracle: the per-edge scores gathered from the field, the pinned
    segment softmax, and the score gradient reduced onto the field's rows."""
    dst = ref.destination_index(rp)
    idx = {"src": col, "dst": dst, "edge": np.arange(col.size)}[role]
    s = scale * np.asarray(table, np.float64)[idx]
    v = np.asarray(value, np.float64)[col]
    out, _ = ref.segment_softmax(rp, s, v)
    ds_e, dv_e = ref.segment_softmax_bwd(rp, s, v, dout)
    dtable = np.zeros(np.asarray(table).shape[0])
    np.add.at(dtable, idx, scale * ds_e)
    dvalue = np.zeros(np.asarray(value).shape, np.float64)
    np.add.at(dvalue, col, dv_e)
    return out, dtable, dvalue


@pytest.mark.parametrize("role,scale", [("src", 1.0), ("edge", 0.5), ("dst", -2.0),
                                        ("edge", 1.0)])
@pytest.mark.parametrize("idx", [torch.int32, torch.int64])
@pytest.mark.parametrize("width", [None, 7])
def test_score_softmax_against_float64(role, scale, idx, width):
    print(f"score softmax role={role} scale={scale} {idx} width={width}", flush=True)
    N = 3000
    rp, col = skewed_csr(31, N, N, mean_deg=9, hubs=(2500, 700), empty_frac=0.1)
    rng = np.random.default_rng(5)
    rows = {"src": N, "dst": N, "edge": col.size}[role]
    table = (rng.standard_normal(rows) * 3).astype(np.float32)
    value = rng.standard_normal((N,) if width is None else (N, width)).astype(np.float32)
    dout = rng.standard_normal((N,) if width is None else (N, width)).astype(np.float32)
    graph = tg.Graph.from_csr(torch.tensor(rp, device=DEV, dtype=idx),
                              torch.tensor(col, device=DEV, dtype=idx), num_src=N)
    t = torch.tensor(table, device=DEV, requires_grad=True)
    v = torch.tensor(value, device=DEV, requires_grad=True)

    class Attn(tg.MessagePassing):
        reducer = tg.online_softmax()

        def edge(self, src, dst, edge):
            fields = {"src": src, "dst": dst, "edge": edge}[role]
            score = fields.s if scale == 1.0 else fields.s * scale
            return self.reducer(score, src.v)

    fields = {"src": {"v": v}, "dst": {}, "edge": {}}
    fields[role]["s"] = t
    k = Attn()
    out = k(graph=graph, **fields)
    assert k.last_variant.backend == "hip"
    out.backward(torch.tensor(dout, device=DEV))
    e_out, e_dt, e_dv = _expected(rp, col, table, role, scale, value, dout)
    assert rel(out.detach().cpu(), e_out) <= 1e-5
    assert rel(v.grad.cpu(), e_dv) <= 1e-5
    if role == "dst":
        # A row-constant score shifts every score of its row alike: the
        # softmax cannot change, so its gradient is zero up to rounding.
        assert float(t.grad.abs().max()) <= 1e-5 * float(np.abs(e_dv).max())
    else:
        assert rel(t.grad.cpu(), e_dt) <= 1e-5
    empty = np.diff(rp) == 0
    assert not out.detach().cpu().numpy()[empty].any()


@pytest.mark.parametrize("dtype,tol", [(torch.bfloat16, 1e-2), (torch.float16, 2e-3)])
@pytest.mark.parametrize("role", ["src", "edge"])
def test_score_softmax_16bit_fields_against_float64(dtype, tol, role):
    """16-bit score fields and values run the same fp32 softmax and sums as
    the reference's oracle (inputs widened, output in the value's type).
    Compared with the fp64 oracle on the 16-bit inputs; the tolerance is the
    output type's rounding (bf16: 2^-8, fp16: 2^-11 relative) with margin."""
    print(f"score softmax {dtype} role={role}", flush=True)
    N = 3000
    rp, col = skewed_csr(37, N, N, mean_deg=9, hubs=(2500,), empty_frac=0.1)
    rng = np.random.default_rng(9)
    rows = {"src": N, "edge": col.size}[role]
    graph = tg.Graph.from_csr(torch.tensor(rp, device=DEV), torch.tensor(col, device=DEV),
                              num_src=N)
    t = torch.tensor(rng.standard_normal(rows) * 3, device=DEV).to(dtype).requires_grad_(True)
    v = torch.tensor(rng.standard_normal((N, 6)), device=DEV).to(dtype).requires_grad_(True)
    dout = torch.tensor(rng.standard_normal((N, 6)), device=DEV).to(dtype)

    class Attn(tg.MessagePassing):
        reducer = tg.online_softmax()

        def edge(self, src, dst, edge):
            return self.reducer({"src": src, "edge": edge}[role].s, src.v)

    fields = {"src": {"v": v}, "edge": {}}
    fields[role]["s"] = t
    k = Attn()
    out = k(graph=graph, dst={}, **fields)
    assert k.last_variant.backend == "hip" and out.dtype == dtype
    out.backward(dout)
    assert t.grad.dtype == dtype and v.grad.dtype == dtype
    f64 = lambda x: x.detach().double().cpu().numpy()
    e_out, e_dt, e_dv = _expected(rp, col, f64(t), role, 1.0, f64(v), f64(dout))
    assert rel(f64(out), e_out) <= tol
    assert rel(f64(v.grad), e_dv) <= tol
    assert rel(f64(t.grad), e_dt) <= tol


@pytest.mark.parametrize("role,scale,width", [("src", 1.0, None), ("edge", 0.5, 8),
                                              ("dst", -2.0, 3), ("src", 1.0, 9)])
@pytest.mark.parametrize("idx", [torch.int32, torch.int64])
def test_score_softmax_without_gradient_against_float64(role, scale, width, idx):
    """Without a gradient the softmax and the value sum run in one pass
    (tgx_segment_softmax_sum_fwd) for fp32 value rows of at most 8 floats;
    9 floats take the softmax weights and the CSR sum.  Hub rows of 2500 and
    700 edges and empty rows; 1e-5 against the float64 oracle; the
    reference's known answer at scores about 1000 too."""
    print(f"score softmax no-grad role={role} scale={scale} width={width} {idx}", flush=True)
    N = 3000
    rp, col = skewed_csr(41, N, N, mean_deg=9, hubs=(2500, 700), empty_frac=0.1)
    rng = np.random.default_rng(11)
    rows = {"src": N, "dst": N, "edge": col.size}[role]
    table = (rng.standard_normal(rows) * 3).astype(np.float32)
    value = rng.standard_normal((N,) if width is None else (N, width)).astype(np.float32)
    graph = tg.Graph.from_csr(torch.tensor(rp, device=DEV, dtype=idx),
                              torch.tensor(col, device=DEV, dtype=idx), num_src=N)

    class Attn(tg.MessagePassing):
        reducer = tg.online_softmax()

        def edge(self, src, dst, edge):
            fields = {"src": src, "dst": dst, "edge": edge}[role]
            return self.reducer(fields.s if scale == 1.0 else fields.s * scale, src.v)

    fields = {"src": {"v": torch.tensor(value, device=DEV)}, "dst": {}, "edge": {}}
    fields[role]["s"] = torch.tensor(table, device=DEV)
    k = Attn()
    with torch.no_grad():
        out = k(graph=graph, **fields)
    assert k.last_variant.backend == "hip"
    e_out, _, _ = _expected(rp, col, table, role, scale, value,
                            np.zeros((N,) if width is None else (N, width)))
    assert rel(out.cpu(), e_out) <= 1e-5
    assert not out.cpu().numpy()[np.diff(rp) == 0].any()
    g = GOLD["online_softmax_large_scores"]
    kg = tg.Graph.from_csr(torch.tensor(g["row_ptr"], device=DEV),
                           torch.tensor(g["col_idx"], device=DEV), num_src=g["num_src"])
    with torch.no_grad():
        o = OnlineAttention()(graph=kg, src={"score": torch.tensor(g["score"], device=DEV),
                                             "value": torch.tensor(g["value"], device=DEV)},
                              dst={})
    np.testing.assert_allclose(o.cpu().numpy(), g["out"], rtol=0,
                               atol=0.5 * 10.0 ** -g["places"])

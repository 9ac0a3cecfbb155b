"""Torch autograd bridges over the HIP kernels.

Outputs and gradients are allocated by Torch on the input's device and every
launch is enqueued on Torch's current stream, as the reference adapter does
(python/tiga/interop/torch/provider.py:8-14, 170-198).  Backward functions
return ``None`` for topology arguments (reference
python/tiga/interop/torch/message_passing.py:193-277, 378-409).
"""

from __future__ import annotations

import ctypes

import torch

from . import _native
from .graph import Graph


def _partial(plan_handle, state_floats: int, device) -> torch.Tensor | None:
    n = plan_handle.plan.n_chunks * state_floats
    if n == 0:
        return None
    return torch.empty(n, dtype=torch.float32, device=device)


def _p(t):
    return None if t is None else t.data_ptr()


class CsrSumFunction(torch.autograd.Function):
    """out[i] = sum_e w[e] * x[col[e]]  (w optional), fp32."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, w: torch.Tensor | None, graph: Graph):
        row_ptr, col_idx = graph._kernel_csr()
        n_dst, n_src = graph.schema.num_dst, graph.schema.num_src
        feat_shape = tuple(x.shape[1:])
        F = 1
        for d in feat_shape:
            F *= d
        xc = x.contiguous()
        wc = None if w is None else w.reshape(-1).contiguous()
        out = torch.empty((n_dst, *feat_shape), dtype=x.dtype, device=x.device)
        if n_dst and F:
            plan = graph._row_plan()
            partial = _partial(plan, F, x.device)
            _native.call("tgx_csr_sum_fwd", row_ptr.data_ptr(), col_idx.data_ptr(),
                         _native.idx_bits(row_ptr), plan.ref, xc.data_ptr(), _p(wc),
                         out.data_ptr(), n_dst, n_src, F, _p(partial), _native.stream_of(x))
        ctx.graph = graph
        ctx.F = F
        ctx.w_shape = None if w is None else w.shape
        ctx.save_for_backward(xc, wc)
        return out

    @staticmethod
    def backward(ctx, dout: torch.Tensor):
        xc, wc = ctx.saved_tensors
        graph: Graph = ctx.graph
        need_dx = ctx.needs_input_grad[0]
        need_dw = wc is not None and ctx.needs_input_grad[1]
        if not (need_dx or need_dw):
            return None, None, None
        n_dst, n_src = graph.schema.num_dst, graph.schema.num_src
        E = graph.num_edges
        dout = dout.contiguous()
        dx = torch.empty_like(xc) if need_dx else None
        dw = torch.empty(E, dtype=xc.dtype, device=xc.device) if need_dw else None
        if n_src and ctx.F and (E or need_dx):
            t = graph._transposed()
            partial = _partial(t.plan, ctx.F, xc.device) if need_dx else None
            _native.call("tgx_csr_sum_bwd", t.row_ptr_t.data_ptr(), t.col_t.data_ptr(),
                         t.perm.data_ptr(), t.plan.ref, xc.data_ptr(), _p(wc),
                         dout.data_ptr(), _p(dx), _p(dw), n_dst, n_src, ctx.F, _p(partial),
                         _native.stream_of(xc))
        if dw is not None:
            dw = dw.reshape(ctx.w_shape)
        return dx, dw, None


class GatFunction(torch.autograd.Function):
    """GAT additive attention: h [N, H, D] fp32, a_src/a_dst [H, D]."""

    @staticmethod
    def forward(ctx, h: torch.Tensor, a_src: torch.Tensor, a_dst: torch.Tensor,
                slope: float, graph: Graph):
        row_ptr, col_idx = graph._kernel_csr()
        N, H, D = h.shape
        hc = h.contiguous()
        asc = a_src.reshape(H, D).contiguous()
        adc = a_dst.reshape(H, D).contiguous()
        out = torch.empty_like(hc)
        ns = torch.empty((N, H, 4), dtype=torch.float32, device=h.device)
        plan = graph._row_plan()
        partial = _partial(plan, H * D + 2 * H, h.device)
        _native.call("tgx_gat_fwd", row_ptr.data_ptr(), col_idx.data_ptr(),
                     _native.idx_bits(row_ptr), plan.ref, hc.data_ptr(), asc.data_ptr(),
                     adc.data_ptr(), float(slope), out.data_ptr(), ns.data_ptr(), N, H, D,
                     _p(partial), _native.stream_of(h))
        ctx.graph = graph
        ctx.slope = float(slope)
        ctx.a_shapes = (a_src.shape, a_dst.shape)
        ctx.save_for_backward(hc, asc, adc, out, ns)
        return out

    @staticmethod
    def backward(ctx, dout: torch.Tensor):
        hc, asc, adc, out, ns = ctx.saved_tensors
        graph: Graph = ctx.graph
        row_ptr, col_idx = graph._kernel_csr()
        N, H, D = hc.shape
        E = graph.num_edges
        dout = dout.contiguous()
        dh = torch.empty_like(hc)
        da_src = torch.empty((H, D), dtype=torch.float32, device=hc.device)
        da_dst = torch.empty((H, D), dtype=torch.float32, device=hc.device)
        plan = graph._row_plan()
        t = graph._transposed()
        ws_bytes = ctypes.c_size_t()
        _native.call("tgx_gat_bwd_workspace", plan.ref, t.plan.ref, E, H, D,
                     ctypes.byref(ws_bytes))
        ws = torch.empty(max(ws_bytes.value, 1), dtype=torch.uint8, device=hc.device)
        # Slot 1 of the saved node state is backward scratch (delta); it is
        # rewritten by every backward before it is read.
        _native.call("tgx_gat_bwd", row_ptr.data_ptr(), col_idx.data_ptr(),
                     _native.idx_bits(row_ptr), plan.ref, t.row_ptr_t.data_ptr(),
                     t.col_t.data_ptr(), t.perm.data_ptr(), t.inv_perm.data_ptr(),
                     t.plan.ref, hc.data_ptr(),
                     asc.data_ptr(), adc.data_ptr(), ctx.slope, out.data_ptr(),
                     ns.data_ptr(), dout.data_ptr(), dh.data_ptr(), da_src.data_ptr(),
                     da_dst.data_ptr(), N, E, H, D, ws.data_ptr(), ws_bytes.value,
                     _native.stream_of(hc))
        return (dh, da_src.reshape(ctx.a_shapes[0]), da_dst.reshape(ctx.a_shapes[1]),
                None, None)


class DotAttnFunction(torch.autograd.Function):
    """Dot-product attention, bf16 q [Nd,H,D], k/v [Ns,H,D], bias [E,H] fp32."""

    @staticmethod
    def forward(ctx, q, k, v, bias, scale: float, graph: Graph):
        row_ptr, col_idx = graph._kernel_csr()
        n_dst, n_src = graph.schema.num_dst, graph.schema.num_src
        _, H, D = q.shape
        qc, kc, vc = q.contiguous(), k.contiguous(), v.contiguous()
        bc = None if bias is None else bias.contiguous()
        out = torch.empty_like(qc)
        ml = torch.empty((n_dst, H, 2), dtype=torch.float32, device=q.device)
        plan = graph._row_plan()
        partial = _partial(plan, H * D + 2 * H, q.device)
        _native.call("tgx_dot_attn_fwd", row_ptr.data_ptr(), col_idx.data_ptr(),
                     _native.idx_bits(row_ptr), plan.ref, qc.data_ptr(), kc.data_ptr(),
                     vc.data_ptr(), _p(bc), float(scale), out.data_ptr(), ml.data_ptr(),
                     n_dst, n_src, H, D, _p(partial), _native.stream_of(q))
        ctx.graph = graph
        ctx.scale = float(scale)
        ctx.has_bias = bias is not None
        ctx.save_for_backward(qc, kc, vc, bc, out, ml)
        return out

    @staticmethod
    def backward(ctx, dout):
        qc, kc, vc, bc, out, ml = ctx.saved_tensors
        graph: Graph = ctx.graph
        row_ptr, col_idx = graph._kernel_csr()
        n_dst, n_src = graph.schema.num_dst, graph.schema.num_src
        _, H, D = qc.shape
        E = graph.num_edges
        dout = dout.contiguous()
        if dout.dtype != qc.dtype:
            dout = dout.to(qc.dtype)
        dq = torch.empty_like(qc)
        dk = torch.empty_like(kc)
        dv = torch.empty_like(vc)
        need_db = ctx.has_bias and ctx.needs_input_grad[3]
        dbias = torch.empty((E, H), dtype=torch.float32, device=qc.device) if need_db else None
        plan = graph._row_plan()
        t = graph._transposed()
        ws_bytes = ctypes.c_size_t()
        _native.call("tgx_dot_attn_bwd_workspace", plan.ref, t.plan.ref, H, D,
                     ctypes.byref(ws_bytes))
        ws = torch.empty(max(ws_bytes.value, 1), dtype=torch.uint8, device=qc.device)
        # Slot 1 of the saved ml is backward scratch (delta), rewritten each time.
        _native.call("tgx_dot_attn_bwd", row_ptr.data_ptr(), col_idx.data_ptr(),
                     _native.idx_bits(row_ptr), plan.ref, t.row_ptr_t.data_ptr(),
                     t.col_t.data_ptr(), t.perm.data_ptr(), t.plan.ref, qc.data_ptr(),
                     kc.data_ptr(), vc.data_ptr(), _p(bc), ctx.scale, out.data_ptr(),
                     ml.data_ptr(), dout.data_ptr(), dq.data_ptr(), dk.data_ptr(),
                     dv.data_ptr(), _p(dbias), n_dst, n_src, H, D, ws.data_ptr(),
                     ws_bytes.value, _native.stream_of(qc))
        return dq, dk, dv, dbias, None, None


class VarlenCausalFunction(torch.autograd.Function):
    """Causal attention on a Graph.cu_seqlens relation: q/k/v [T, H, 128] bf16."""

    @staticmethod
    def forward(ctx, q, k, v, scale: float, graph: Graph):
        T, H, D = q.shape
        qc, kc, vc = q.contiguous(), k.contiguous(), v.contiguous()
        cu, tasks, n = graph._varlen_tasks(0, 128, H)
        out = torch.empty_like(qc)
        lse = torch.empty((T, H), dtype=torch.float32, device=q.device)
        _native.call("tgx_varlen_causal_fwd", cu.data_ptr(), tasks.data_ptr(), n,
                     qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), float(scale), out.data_ptr(),
                     lse.data_ptr(), T, H, D, _native.stream_of(q))
        ctx.graph = graph
        ctx.scale = float(scale)
        ctx.save_for_backward(qc, kc, vc, out, lse)
        return out

    @staticmethod
    def backward(ctx, dout):
        qc, kc, vc, out, lse = ctx.saved_tensors
        graph: Graph = ctx.graph
        T, H, D = qc.shape
        dout = dout.contiguous()
        if dout.dtype != qc.dtype:
            dout = dout.to(qc.dtype)
        cu, qtasks, nq = graph._varlen_tasks(0, 128, H)
        _, ktasks, nk = graph._varlen_tasks(1, 64, H)
        dq, dk, dv = torch.empty_like(qc), torch.empty_like(kc), torch.empty_like(vc)
        delta = torch.empty((T, H), dtype=torch.float32, device=qc.device)
        _native.call("tgx_varlen_causal_bwd", cu.data_ptr(), qtasks.data_ptr(), nq,
                     ktasks.data_ptr(), nk, qc.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                     out.data_ptr(), lse.data_ptr(), dout.data_ptr(), ctx.scale, dq.data_ptr(),
                     dk.data_ptr(), dv.data_ptr(), delta.data_ptr(), T, H, D,
                     _native.stream_of(qc))
        return dq, dk, dv, None, None

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


_ATTN_DTYPES = {torch.bfloat16: 0, torch.float16: 1}


def attn_strides(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor):
    """(q, k, v, strides) with the innermost dim dense and k, v sharing
    token/head strides, as the attention tiles read them: contiguous
    [n, H, D], or [H, n, D] storage viewed as [n, H, D] (the layout of the
    reference's dense streaming path, message_passing.py:1944-1947), are
    used in place; anything else is made contiguous."""
    if q.stride(-1) != 1 or min(q.stride(0), q.stride(1)) <= 0:
        q = q.contiguous()
    if k.stride(-1) != 1 or v.stride() != k.stride() or min(k.stride(0), k.stride(1)) <= 0:
        k, v = k.contiguous(), v.contiguous()
    strides = (ctypes.c_int64 * 4)(q.stride(0), q.stride(1), k.stride(0), k.stride(1))
    return q, k, v, strides


class BlockAttentionFunction(torch.autograd.Function):
    """Dot-product attention over a block-diagonal relation: Graph.cu_seqlens
    (causal or not), Graph.dense, Graph.triangular.  q [n_dst, H, D], k/v
    [n_src, H, D], bf16 or fp16, D in {64, 128}; out contiguous [n_dst, H, D].
    prune > 0 is the reference's block_prune_threshold (forward only)."""

    @staticmethod
    def forward(ctx, q, k, v, scale: float, prune: float, graph: Graph):
        n_q, H, D = q.shape
        n_k = k.shape[0]
        q, k, v, strides = attn_strides(q, k, v)
        cu_q, cu_k, tasks, n, causal = graph._attn_tasks(0, 128, H)
        out = torch.empty((n_q, H, D), dtype=q.dtype, device=q.device)
        lse = torch.empty((n_q, H), dtype=torch.float32, device=q.device)
        _native.call("tgx_attn_fwd", cu_q.data_ptr(), cu_k.data_ptr(), tasks.data_ptr(), n,
                     int(causal), _ATTN_DTYPES[q.dtype], q.data_ptr(), k.data_ptr(),
                     v.data_ptr(), strides, float(scale), float(prune), out.data_ptr(),
                     lse.data_ptr(), n_q, n_k, H, D, _native.stream_of(q))
        ctx.graph = graph
        ctx.scale = float(scale)
        ctx.pruned = prune > 0
        ctx.save_for_backward(q, k, v, out, lse)
        return out

    @staticmethod
    def backward(ctx, dout):
        if ctx.pruned:
            raise NotImplementedError(
                "block_prune_threshold is a forward-only approximation: it has no gradient")
        q, k, v, out, lse = ctx.saved_tensors
        graph: Graph = ctx.graph
        n_q, H, D = q.shape
        n_k = k.shape[0]
        dout = dout.contiguous()
        if dout.dtype != q.dtype:
            dout = dout.to(q.dtype)
        strides = attn_strides(q, k, v)[3]   # saved tensors already have tile strides
        cu_q, cu_k, qtasks, nq, causal = graph._attn_tasks(0, 128, H)
        _, _, ktasks, nk, _ = graph._attn_tasks(1, 64, H)
        dq = torch.empty((n_q, H, D), dtype=q.dtype, device=q.device)
        dk = torch.empty((n_k, H, D), dtype=q.dtype, device=q.device)
        dv = torch.empty((n_k, H, D), dtype=q.dtype, device=q.device)
        delta = torch.empty((n_q, H), dtype=torch.float32, device=q.device)
        _native.call("tgx_attn_bwd", cu_q.data_ptr(), cu_k.data_ptr(), qtasks.data_ptr(), nq,
                     ktasks.data_ptr(), nk, int(causal), _ATTN_DTYPES[q.dtype], q.data_ptr(),
                     k.data_ptr(), v.data_ptr(), strides, out.data_ptr(), lse.data_ptr(),
                     dout.data_ptr(), ctx.scale, dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                     delta.data_ptr(), n_q, n_k, H, D, _native.stream_of(q))
        return dq, dk, dv, None, None, None


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


def _on_graph_device(graph: Graph, *tensors) -> None:
    """Every operand of a launch must live on the graph's device: the kernels
    dereference raw pointers, and a host pointer would fault the GPU."""
    device = graph.device
    for t in tensors:
        if t is not None and t.device != device:
            raise ValueError(f"operand on {t.device} for a graph on {device}")


def _aligned(t: torch.Tensor) -> torch.Tensor:
    """Contiguous with a 16-byte aligned start (the kernels' vector loads)."""
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _csr_sum_launch(x: torch.Tensor, w: torch.Tensor | None, graph: Graph):
    """The forward launch of tg.sum() of [w *] x: (out, x and w as the
    kernel read them, F)."""
    _on_graph_device(graph, x, w)
    row_ptr, col_idx = graph._kernel_csr()
    n_dst, n_src = graph.schema.num_dst, graph.schema.num_src
    feat_shape = tuple(x.shape[1:])
    F = 1
    for d in feat_shape:
        F *= d
    xc = _aligned(x)
    wc = None if w is None else w.reshape(-1).contiguous()
    out = torch.empty((n_dst, *feat_shape), dtype=x.dtype, device=x.device)
    if n_dst and F:
        plan = graph._row_plan()
        partial = _partial(plan, F, x.device)
        _native.call("tgx_csr_sum_fwd", row_ptr.data_ptr(), col_idx.data_ptr(),
                     _native.idx_bits(row_ptr), plan.ref, xc.data_ptr(), _p(wc),
                     out.data_ptr(), n_dst, n_src, F, _native.dtype_code(xc), _p(partial),
                     _native.stream_of(x))
    return out, xc, wc, F


def csr_sum(x: torch.Tensor, w: torch.Tensor | None, graph: Graph) -> torch.Tensor:
    """tg.sum() of [w *] x with autograd when an operand needs a gradient,
    else the bare launch (no autograd node: the prepared and no-grad calls'
    host cost is the launch's own)."""
    if torch.is_grad_enabled() and (x.requires_grad or (w is not None and w.requires_grad)):
        return CsrSumFunction.apply(x, w, graph)
    return _csr_sum_launch(x, w, graph)[0]


def bind_csr_sum(x: torch.Tensor, w: torch.Tensor | None, graph: Graph):
    """The forward launch of tg.sum() of [w *] x with every native argument
    but the output bound: a zero-argument callable returning a new output
    per call, or None when the kernel would not read x and w in place (a
    converted or compacted copy would hide later in-place updates)."""
    _on_graph_device(graph, x, w)
    xc = _aligned(x)
    wc = None if w is None else w.reshape(-1).contiguous()
    if xc.data_ptr() != x.data_ptr() or (wc is not None and wc.data_ptr() != w.data_ptr()):
        return None
    row_ptr, col_idx = graph._kernel_csr()
    n_dst, n_src = graph.schema.num_dst, graph.schema.num_src
    feat_shape = tuple(x.shape[1:])
    F = 1
    for d in feat_shape:
        F *= d
    out_shape, dtype, device = (n_dst, *feat_shape), x.dtype, x.device
    if not (n_dst and F):
        return lambda: torch.empty(out_shape, dtype=dtype, device=device)
    plan = graph._row_plan()
    n_partial = plan.plan.n_chunks * F   # split-row partials: fresh per call
    fn = _native.lib().tgx_csr_sum_fwd
    head = (row_ptr.data_ptr(), col_idx.data_ptr(), _native.idx_bits(row_ptr), plan.ref,
            xc.data_ptr(), _p(wc))
    tail = (n_dst, n_src, F, _native.dtype_code(xc))
    keep = (row_ptr, col_idx, plan, xc, wc)   # alive as long as the launch
    index = device.index if device.index is not None else torch.cuda.current_device()
    raw_stream = torch._C._cuda_getCurrentRawStream

    def launch():
        out = torch.empty(out_shape, dtype=dtype, device=device)
        partial = (torch.empty(n_partial, dtype=torch.float32, device=device)
                   if n_partial else None)
        status = fn(*head, out.data_ptr(), *tail, _p(partial), raw_stream(index))
        if status != 0:
            _native.raise_status("tgx_csr_sum_fwd", status)
        return out

    launch.keep = keep
    return launch


class CsrSumFunction(torch.autograd.Function):
    """out[i] = sum_e w[e] * x[col[e]]  (w optional): x fp32, bf16 or fp16
    (out, dout and dx of the same type), w fp32; fp32 products and sums."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, w: torch.Tensor | None, graph: Graph):
        out, xc, wc, F = _csr_sum_launch(x, w, graph)
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
        dout = _aligned(dout.to(xc.dtype))
        dx = torch.empty_like(xc) if need_dx else None
        dw = torch.empty(E, dtype=torch.float32, device=xc.device) if need_dw else None
        # Narrow rows (F <= 32): dw in edge order from a pass over the CSR
        # (contiguous writes) instead of scattered through the transpose.
        dw_in_csr = dw is not None and ctx.F <= 32 and E > 0
        if n_src and ctx.F and (need_dx or (E and not dw_in_csr)):
            t = graph._transposed()
            partial = _partial(t.plan, ctx.F, xc.device) if need_dx else None
            _native.call("tgx_csr_sum_bwd", t.row_ptr_t.data_ptr(), t.col_t.data_ptr(),
                         t.perm.data_ptr(), t.plan.ref, xc.data_ptr(), _p(wc),
                         dout.data_ptr(), _p(dx), None if dw_in_csr else _p(dw), n_dst,
                         n_src, ctx.F, _native.dtype_code(xc), _p(partial),
                         _native.stream_of(xc))
        if dw_in_csr:
            row_ptr, col_idx = graph._kernel_csr()
            _native.call("tgx_csr_edge_dot", row_ptr.data_ptr(), col_idx.data_ptr(),
                         _native.idx_bits(row_ptr), graph._row_plan().ref, xc.data_ptr(),
                         dout.data_ptr(), dw.data_ptr(), n_dst, n_src, ctx.F,
                         _native.dtype_code(xc), _native.stream_of(xc))
        if dw is not None:
            dw = dw.reshape(ctx.w_shape)
        return dx, dw, None


class GatFunction(torch.autograd.Function):
    """GAT additive attention: source features h_src [Ns, H, D] and
    destination features h_dst [Nd, H, D] (None: h_src serves both roles of
    a homogeneous relation) of one element type (fp32, bf16 or fp16; fp32
    arithmetic, outputs in that type), a_src/a_dst fp32 [H, D]."""

    @staticmethod
    def forward(ctx, h_src: torch.Tensor, h_dst, a_src: torch.Tensor, a_dst: torch.Tensor,
                slope: float, graph: Graph):
        _on_graph_device(graph, h_src, h_dst, a_src, a_dst)
        row_ptr, col_idx = graph._kernel_csr()
        n_dst, n_src = graph.schema.num_dst, graph.schema.num_src
        _, H, D = h_src.shape
        hs = _aligned(h_src)
        hd = hs if h_dst is None else _aligned(h_dst)
        asc = _aligned(a_src.reshape(H, D))
        adc = _aligned(a_dst.reshape(H, D))
        out = torch.empty((n_dst, H, D), dtype=hs.dtype, device=hs.device)
        ns = torch.empty((n_dst, H, 4), dtype=torch.float32, device=hs.device)
        # A forward that a backward may follow also writes pos, each row's
        # sum over its z > 0 edges of alpha (h[j] - out[i]): the backward
        # then forms the destination terms from node rows instead of a
        # per-edge pass.
        pos = (torch.empty((n_dst, H, D), dtype=torch.float32, device=hs.device)
               if any(ctx.needs_input_grad[:4]) else None)
        plan = graph._row_plan()
        partial = _partial(plan, 2 * H * D + 3 * H if pos is not None else H * D + 2 * H,
                           hs.device)
        _native.call("tgx_gat_fwd", row_ptr.data_ptr(), col_idx.data_ptr(),
                     _native.idx_bits(row_ptr), plan.ref, hs.data_ptr(), hd.data_ptr(),
                     asc.data_ptr(), adc.data_ptr(), float(slope), out.data_ptr(),
                     ns.data_ptr(), n_dst, n_src, H, D, _VALUE_DTYPES[hs.dtype], _p(partial),
                     _p(pos), _native.stream_of(hs))
        ctx.graph = graph
        ctx.slope = float(slope)
        ctx.a_shapes = (a_src.shape, a_dst.shape)
        ctx.bipartite = h_dst is not None
        ctx.save_for_backward(hs, hd, asc, adc, out, pos, ns)
        return out

    @staticmethod
    def backward(ctx, dout: torch.Tensor):
        hs, hd, asc, adc, out, pos, ns = ctx.saved_tensors
        graph: Graph = ctx.graph
        row_ptr, col_idx = graph._kernel_csr()
        n_dst, n_src = graph.schema.num_dst, graph.schema.num_src
        _, H, D = hs.shape
        E = graph.num_edges
        dout = _aligned(dout.to(hs.dtype))
        dh_src = torch.empty_like(hs)
        dh_dst = torch.empty_like(hd) if ctx.bipartite else dh_src
        da_src = torch.empty((H, D), dtype=torch.float32, device=hs.device)
        da_dst = torch.empty((H, D), dtype=torch.float32, device=hs.device)
        plan = graph._row_plan()
        t = graph._transposed()
        code = _VALUE_DTYPES[hs.dtype]
        ws_bytes = ctypes.c_size_t()
        _native.call("tgx_gat_bwd_workspace", plan.ref, t.plan.ref, E, H, D, code,
                     int(pos is not None), ctypes.byref(ws_bytes))
        ws = torch.empty(max(ws_bytes.value, 1), dtype=torch.uint8, device=hs.device)
        # Slot 1 of the saved node state is backward scratch (delta); it is
        # rewritten by every backward before it is read.
        _native.call("tgx_gat_bwd", row_ptr.data_ptr(), col_idx.data_ptr(),
                     _native.idx_bits(row_ptr), plan.ref, t.row_ptr_t.data_ptr(),
                     t.col_t.data_ptr(), t.perm.data_ptr(), t.inv_perm.data_ptr(),
                     t.plan.ref, hs.data_ptr(), hd.data_ptr(), asc.data_ptr(), adc.data_ptr(),
                     ctx.slope, out.data_ptr(), ns.data_ptr(), _p(pos), dout.data_ptr(),
                     dh_src.data_ptr(), dh_dst.data_ptr(), da_src.data_ptr(),
                     da_dst.data_ptr(), n_dst, n_src, E, H, D, code, ws.data_ptr(),
                     ws_bytes.value, _native.stream_of(hs))
        return (dh_src, dh_dst if ctx.bipartite else None, da_src.reshape(ctx.a_shapes[0]),
                da_dst.reshape(ctx.a_shapes[1]), None, None)


# Element types of the CSR dot-product and GAT kernels (TGX_DTYPE_*).
_VALUE_DTYPES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


class DotAttnFunction(torch.autograd.Function):
    """Dot-product attention: q [Nd,H,D], k/v [Ns,H,D] of one element type
    (bf16, fp16 or fp32; fp32 arithmetic, output in that type), bias [E,H]
    fp32."""

    @staticmethod
    def forward(ctx, q, k, v, bias, scale: float, graph: Graph):
        _on_graph_device(graph, q, k, v, bias)
        row_ptr, col_idx = graph._kernel_csr()
        n_dst, n_src = graph.schema.num_dst, graph.schema.num_src
        _, H, D = q.shape
        qc, kc, vc = _aligned(q), _aligned(k), _aligned(v)
        bc = None if bias is None else bias.contiguous()
        out = torch.empty_like(qc)
        ml = torch.empty((n_dst, H, 2), dtype=torch.float32, device=q.device)
        plan = graph._row_plan()
        partial = _partial(plan, H * D + 2 * H, q.device)
        _native.call("tgx_dot_attn_fwd", row_ptr.data_ptr(), col_idx.data_ptr(),
                     _native.idx_bits(row_ptr), plan.ref, qc.data_ptr(), kc.data_ptr(),
                     vc.data_ptr(), _p(bc), float(scale), out.data_ptr(), ml.data_ptr(),
                     n_dst, n_src, H, D, _VALUE_DTYPES[qc.dtype], _p(partial),
                     _native.stream_of(q))
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
        dout = _aligned(dout.to(qc.dtype))
        dq = torch.empty_like(qc)
        dk = torch.empty_like(kc)
        dv = torch.empty_like(vc)
        need_db = ctx.has_bias and ctx.needs_input_grad[3]
        dbias = torch.empty((E, H), dtype=torch.float32, device=qc.device) if need_db else None
        plan = graph._row_plan()
        t = graph._transposed()
        ws_bytes = ctypes.c_size_t()
        # Stored ds: the source pass keeps each edge's score gradient for the
        # destination pass, which then gathers only k rows.
        _native.call("tgx_dot_attn_bwd_workspace", plan.ref, t.plan.ref, E, H, D, 1,
                     ctypes.byref(ws_bytes))
        ws = torch.empty(max(ws_bytes.value, 1), dtype=torch.uint8, device=qc.device)
        # Slot 1 of the saved ml is backward scratch (delta), rewritten each time.
        _native.call("tgx_dot_attn_bwd", row_ptr.data_ptr(), col_idx.data_ptr(),
                     _native.idx_bits(row_ptr), plan.ref, t.row_ptr_t.data_ptr(),
                     t.col_t.data_ptr(), t.perm.data_ptr(), t.inv_perm.data_ptr(), t.plan.ref,
                     E, qc.data_ptr(),
                     kc.data_ptr(), vc.data_ptr(), _p(bc), ctx.scale, out.data_ptr(),
                     ml.data_ptr(), dout.data_ptr(), dq.data_ptr(), dk.data_ptr(),
                     dv.data_ptr(), _p(dbias), n_dst, n_src, H, D, _VALUE_DTYPES[qc.dtype],
                     ws.data_ptr(), ws_bytes.value, _native.stream_of(qc))
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


# The attention backward stores dS (tgx_attn_bwd_stored: the dQ pass reads
# it back instead of recomputing S and dP) when its workspace is at most this
# many bytes; larger relations recompute (tgx_attn_bwd).
STORED_DS_MAX_BYTES = 8 << 30
# Keys per dK/dV workgroup of the attention backward (the key task lists of
# tgx_attn_tasks, kind 1, are built with this block).
ATTN_KEY_TILE = 64


class BlockAttentionFunction(torch.autograd.Function):
    """Dot-product attention over a block-diagonal relation: Graph.cu_seqlens
    (causal or not), Graph.dense, Graph.triangular.  q [n_dst, H, D], k/v
    [n_src, H, D], bf16 or fp16, D in {32, 64, 128}; out contiguous [n_dst, H, D].
    prune > 0 is the reference's block_prune_threshold (forward only)."""

    @staticmethod
    def forward(ctx, q, k, v, scale: float, prune: float, graph: Graph):
        _on_graph_device(graph, q, k, v)
        n_q, H, D = q.shape
        n_k = k.shape[0]
        q, k, v, strides = attn_strides(q, k, v)
        cu_q, cu_k, tasks, n, causal = graph._attn_tasks(0, 128, H)
        out = torch.empty((n_q, H, D), dtype=q.dtype, device=q.device)
        lse = torch.empty((n_q, H), dtype=torch.float32, device=q.device)
        split = None if prune > 0 else graph._attn_fwd_split(H)
        if split is not None:
            # Too few, too uneven query tiles: the longest key ranges run in
            # chunks, merged afterwards (tgx_attn_fwd_split).
            stasks, sn, merge, n_merge, chunk, max_chunks = split
            partial = torch.empty(n_merge * max_chunks * 128 * (D + 2), dtype=torch.float32,
                                  device=q.device)
            _native.call("tgx_attn_fwd_split", cu_q.data_ptr(), cu_k.data_ptr(),
                         stasks.data_ptr(), sn, merge.data_ptr(), n_merge, chunk, max_chunks,
                         int(causal), _ATTN_DTYPES[q.dtype], q.data_ptr(), k.data_ptr(),
                         v.data_ptr(), strides, float(scale), out.data_ptr(), lse.data_ptr(),
                         partial.data_ptr(), n_q, n_k, H, D, _native.stream_of(q))
        else:
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
        _, _, ktasks, nk, _ = graph._attn_tasks(1, ATTN_KEY_TILE, H)
        dq = torch.empty((n_q, H, D), dtype=q.dtype, device=q.device)
        dk = torch.empty((n_k, H, D), dtype=q.dtype, device=q.device)
        dv = torch.empty((n_k, H, D), dtype=q.dtype, device=q.device)
        delta = torch.empty((n_q, H), dtype=torch.float32, device=q.device)
        args = (cu_q.data_ptr(), cu_k.data_ptr(), qtasks.data_ptr(), nq, ktasks.data_ptr(), nk,
                int(causal), _ATTN_DTYPES[q.dtype], q.data_ptr(), k.data_ptr(), v.data_ptr(),
                strides, out.data_ptr(), lse.data_ptr(), dout.data_ptr(), ctx.scale,
                dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), delta.data_ptr())
        tail = (n_q, n_k, H, D, _native.stream_of(q))
        tiles = graph._attn_ds_tiles(H)
        if tiles is not None and tiles * 64 * 64 * q.element_size() <= STORED_DS_MAX_BYTES:
            ds = torch.empty(max(tiles, 1) * 64 * 64, dtype=q.dtype, device=q.device)
            _native.call("tgx_attn_bwd_stored", *args, ds.data_ptr(), *tail)
        else:
            _native.call("tgx_attn_bwd", *args, *tail)
        return dq, dk, dv, None, None, None



# ---------------------------------------------------------------------------
# nn-scored edge attention (tgx_nn.hip)

_ROLE = {"src": 0, "dst": 1, "edge": 2}


def _padded_width(chain, in_width: int, vector: bool = False) -> int:
    """The common padded width of a chain's layers: every input and output
    width, except the last layer's output for an edge-network sum (the
    kernels never evaluate that layer)."""
    outs = [l.linear.out_features for l in (chain[:-1] if vector else chain)]
    widest = max([in_width] + [l.linear.in_features for l in chain] + outs)
    return next(w for w in (16, 24, 32, 64) if w >= widest)


def _folded(layer, weight, bias):
    """The folded weights of one layer, z = W' a + b', with the scalar maps
    on its input (in_scale, in_shift) and output (scale, shift):
    W' = scale in_scale W, b' = scale (b + in_shift W 1) + shift.  b' is
    None when it is identically zero."""
    w = weight.detach()
    f = layer.scale * layer.in_scale
    # (Factors of 1 are skipped: each product is a launch of its own.)
    wf = w if f == 1.0 else w * f
    bf = None if bias is None else (bias.detach() if layer.scale == 1.0
                                    else bias.detach() * layer.scale)
    if layer.in_shift != 0.0:
        extra = w.sum(1) * (layer.scale * layer.in_shift)
        bf = extra if bf is None else bf + extra
    if layer.shift != 0.0:
        bf = torch.full_like(wf[:, 0], layer.shift) if bf is None else bf + layer.shift
    return wf, bf


def _unfolded_grads(layer, dwf, dbf, need_w, need_b):
    """Gradients of a layer's own weight and bias from those of its folded
    weights W', b' (see _folded): dW = scale in_scale dW' + scale in_shift
    db' 1^T, db = scale db'."""
    dW = db = None
    if need_w and dwf is not None:
        f = layer.scale * layer.in_scale
        dW = dwf if f == 1.0 else dwf * f
        if layer.in_shift != 0.0:
            dW = dW + (dbf * (layer.scale * layer.in_shift))[:, None]
    if need_b and dbf is not None:
        db = dbf if layer.scale == 1.0 else dbf * layer.scale
    return dW, db


def _folded_norm(layer, gamma, beta):
    """A LayerNorm's folded gamma', beta' (the scalar map between it and the
    activation, c y + d, folded in: gamma' = c gamma, beta' = c beta + d)."""
    n = layer.linear.out_features
    like = layer.linear.weight
    g = torch.ones(n, dtype=like.dtype, device=like.device) if gamma is None else gamma.detach()
    b = torch.zeros(n, dtype=like.dtype, device=like.device) if beta is None else beta.detach()
    return g * layer.norm_scale, b * layer.norm_scale + layer.norm_shift


def _block_floats(chain, W: int) -> int:
    """Floats per layer of the weight blocks: [W*W | W bias], and [W gamma |
    W beta] after them when some layer has a LayerNorm."""
    return W * W + W + (2 * W if any(l.norm is not None for l in chain) else 0)


# Parameters per layer passed to the autograd functions: Linear weight and
# bias, LayerNorm weight and bias (None where absent).
_PER_LAYER = 4


def _layer_params(chain):
    params = []
    for layer in chain:
        norm = layer.norm
        params += [layer.linear.weight, layer.linear.bias,
                   None if norm is None else norm.weight, None if norm is None else norm.bias]
    return params


def _fill_weights(buf, chain, params, W, layers):
    """Padded blocks of the folded weights (_folded, _folded_norm) of
    `layers` (buf: [layers or more, _block_floats])."""
    for l in range(layers):
        k = _PER_LAYER * l
        wf, bf = _folded(chain[l], params[k], params[k + 1])
        out_f, in_f = wf.shape
        buf[l, :W * W].view(W, W)[:out_f, :in_f] = wf
        if bf is not None:
            buf[l, W * W:W * W + out_f] = bf
        if chain[l].norm is not None:
            g, b = _folded_norm(chain[l], params[k + 2], params[k + 3])
            buf[l, W * W + W:W * W + W + out_f] = g
            buf[l, W * W + 2 * W:W * W + 2 * W + out_f] = b


def _mlp_struct(chain, roles, segs, weights_buf, width):
    from .nn import _ACT

    m = _native.EdgeMlp()
    m.n_layers = len(chain)
    m.width = width
    for l, layer in enumerate(chain):
        m.act[l] = _ACT[layer.act]
        m.act_param[l] = layer.param
        m.act_param2[l] = layer.param2
        if layer.norm is not None:
            m.norm[l] = 1
            m.norm_eps[l] = float(layer.norm.eps)
        # The last layer of an edge-network sum is applied by the caller;
        # the kernels see it as a one-output layer they do not evaluate.
        m.out_width[l] = layer.linear.out_features if l + 1 < len(chain) else 1
    m.weights_dev = weights_buf.data_ptr()
    m.n_segments = len(segs)
    for s, (role, seg) in enumerate(zip(roles, segs)):
        m.seg_role[s] = _ROLE[role]
        m.seg_width[s] = seg.shape[1]
        m.seg_stride[s] = seg.stride(0)
        m.seg_dev[s] = seg.data_ptr()
    return m


def _as_rows(t: torch.Tensor) -> torch.Tensor:
    """A field as [rows, width] fp32 with unit column stride."""
    t2 = t.reshape(t.shape[0], -1) if t.ndim != 2 else t
    if t2.stride(-1) != 1 or t2.stride(0) < t2.shape[1]:
        t2 = t2.contiguous()
    return t2


class EdgeMlpFunction(torch.autograd.Function):
    """scores[e] = net(concat of the fields gathered for edge e).

    Inputs after (graph, chain, roles, n_seg): the n_seg field tensors, then
    per layer the Linear weight and bias and the LayerNorm weight and bias
    (None allowed)."""

    @staticmethod
    def forward(ctx, graph: Graph, chain, roles, n_seg: int, *tensors):
        _on_graph_device(graph, *tensors)
        segs = [_as_rows(t) for t in tensors[:n_seg]]
        params = tensors[n_seg:]
        row_ptr, col_idx = graph._kernel_csr()
        E = col_idx.numel()
        in_width = sum(s.shape[1] for s in segs)
        W = _padded_width(chain, in_width)
        dev = col_idx.device
        buf = torch.zeros(len(chain), _block_floats(chain, W), dtype=torch.float32, device=dev)
        _fill_weights(buf, chain, params, W, len(chain))
        mlp = _mlp_struct(chain, roles, segs, buf, W)
        scores = torch.empty(E, dtype=torch.float32, device=dev)
        _native.call("tgx_edge_mlp_scores", col_idx.data_ptr(), graph._dst_index32().data_ptr(),
                     _native.idx_bits(row_ptr), E, ctypes.byref(mlp), scores.data_ptr(),
                     _native.stream_of(col_idx))
        ctx.graph, ctx.chain, ctx.roles, ctx.n_seg, ctx.W = graph, chain, roles, n_seg, W
        ctx.shapes = [t.shape for t in tensors[:n_seg]]
        ctx.present = [t is not None for t in params]
        ctx.save_for_backward(buf, *segs)
        return scores

    @staticmethod
    def backward(ctx, dscore):
        buf, *segs = ctx.saved_tensors
        graph, chain, roles, W = ctx.graph, ctx.chain, ctx.roles, ctx.W
        row_ptr, col_idx = graph._kernel_csr()
        E = col_idx.numel()
        dev = col_idx.device
        L = len(chain)
        dscore = dscore.contiguous()
        dsegs = [torch.empty(E, s.shape[1], dtype=torch.float32, device=dev) for s in segs]
        mlp = _mlp_struct(chain, roles, segs, buf, W)
        ws_bytes = ctypes.c_size_t()
        _native.call("tgx_edge_mlp_backward_workspace", E, ctypes.byref(mlp),
                     ctypes.byref(ws_bytes))
        ws = torch.empty(max(ws_bytes.value, 4), dtype=torch.uint8, device=dev)
        dweights = torch.empty(L, buf.shape[1], dtype=torch.float32, device=dev)
        ptrs = (ctypes.c_void_p * 4)(*[d.data_ptr() for d in dsegs], *([None] * (4 - len(dsegs))))
        _native.call("tgx_edge_mlp_backward", col_idx.data_ptr(),
                     graph._dst_index32().data_ptr(), _native.idx_bits(row_ptr), E,
                     ctypes.byref(mlp), dscore.data_ptr(), dweights.data_ptr(), ptrs,
                     ws.data_ptr(), ws_bytes.value, _native.stream_of(col_idx))
        grads = _segment_grads(graph, roles, dsegs, ctx.shapes, ctx.needs_input_grad, 4)
        grads += _layer_grads(chain, dweights, W, ctx.present, ctx.needs_input_grad,
                              4 + ctx.n_seg, len(chain))
        return (None, None, None, None, *grads)


def _layer_grads(chain, dweights, W, present, needs, first, layers):
    """Gradients of the module's own parameters (per layer: Linear weight and
    bias, LayerNorm weight and bias) from the folded blocks' sums
    (_unfolded_grads; d gamma = c d gamma', d beta = c d beta' for the scalar
    map c y + d after the LayerNorm)."""
    grads = []
    for l in range(layers):
        layer = chain[l]
        out_f, in_f = layer.linear.out_features, layer.linear.in_features
        j = _PER_LAYER * l
        k = first + j
        blk = dweights[l]
        grads += list(_unfolded_grads(layer, blk[:W * W].view(W, W)[:out_f, :in_f],
                                      blk[W * W:W * W + out_f], needs[k],
                                      present[j + 1] and needs[k + 1]))
        dg = db = None
        if layer.norm is not None:
            if present[j + 2] and needs[k + 2]:
                dg = blk[W * W + W:W * W + W + out_f] * layer.norm_scale
            if present[j + 3] and needs[k + 3]:
                db = blk[W * W + 2 * W:W * W + 2 * W + out_f] * layer.norm_scale
        grads += [dg, db]
    return grads


def _segment_grads(graph, roles, dsegs, shapes, needs, first):
    """Per-edge input-segment gradients reduced onto their fields' rows."""
    grads = []
    for s, (role, d, shape) in enumerate(zip(roles, dsegs, shapes)):
        if not needs[first + s]:
            grads.append(None)
            continue
        if role == "edge":
            g = d
        elif role == "src":
            g = _reduce_rows_transposed(graph, d)
        else:
            g = _reduce_rows(graph, d)
        grads.append(g.reshape(shape))
    return grads


def _reduce_rows(graph: Graph, x: torch.Tensor) -> torch.Tensor:
    """out[i] = sum of x[e] over the edges e of destination row i (CSR sum
    with the edge ids as columns)."""
    row_ptr, _ = graph._kernel_csr()
    n_dst, E = graph.schema.num_dst, x.shape[0]
    F = x.shape[1]
    out = torch.empty(n_dst, F, dtype=torch.float32, device=x.device)
    if n_dst:
        plan = graph._row_plan()
        partial = _partial(plan, F, x.device)
        _native.call("tgx_csr_sum_fwd", row_ptr.data_ptr(), None,
                     _native.idx_bits(row_ptr), plan.ref, x.data_ptr(), None, out.data_ptr(),
                     n_dst, E, F, _native.DTYPE_F32, _p(partial), _native.stream_of(x))
    return out


def _reduce_rows_transposed(graph: Graph, x: torch.Tensor) -> torch.Tensor:
    """out[j] = sum of x[e] over the edges e whose source is j (CSR sum over
    the transposed CSR with perm as columns)."""
    t = graph._transposed()
    n_src, E, F = graph.schema.num_src, x.shape[0], x.shape[1]
    out = torch.empty(n_src, F, dtype=torch.float32, device=x.device)
    if n_src:
        partial = _partial(t.plan, F, x.device)
        _native.call("tgx_csr_sum_fwd", t.row_ptr_t.data_ptr(), t.perm.data_ptr(), 32,
                     t.plan.ref, x.data_ptr(), None, out.data_ptr(), n_src, E, F,
                     _native.DTYPE_F32, _p(partial), _native.stream_of(x))
    return out


class SegmentSoftmaxFunction(torch.autograd.Function):
    """alpha[e] = softmax of the scores over the edges of each CSR row."""

    @staticmethod
    def forward(ctx, scores: torch.Tensor, graph: Graph):
        _on_graph_device(graph, scores)
        row_ptr, _ = graph._kernel_csr()
        n = graph.schema.num_dst
        alpha = torch.empty_like(scores)
        lse = torch.empty(max(n, 1), dtype=torch.float32, device=scores.device)
        _native.call("tgx_segment_softmax_fwd", row_ptr.data_ptr(), _native.idx_bits(row_ptr),
                     n, scores.data_ptr(), alpha.data_ptr(), lse.data_ptr(),
                     _native.stream_of(scores))
        ctx.graph = graph
        ctx.save_for_backward(alpha)
        return alpha

    @staticmethod
    def backward(ctx, dalpha):
        (alpha,) = ctx.saved_tensors
        graph = ctx.graph
        row_ptr, _ = graph._kernel_csr()
        dalpha = dalpha.contiguous()
        dscore = torch.empty_like(alpha)
        _native.call("tgx_segment_softmax_bwd", row_ptr.data_ptr(), _native.idx_bits(row_ptr),
                     graph.schema.num_dst, alpha.data_ptr(), dalpha.data_ptr(),
                     dscore.data_ptr(), _native.stream_of(alpha))
        return dscore, None


class NnAttentionFunction(torch.autograd.Function):
    """out[i] = sum_e softmax_i(net(fields_e)) value[col[e]], fp32, with the
    logsumexp-recompute backward.  The forward keeps per destination row only
    the logsumexp of its scores and its output (no per-edge score or weight
    outlives it); the backward replays the network per edge and forms alpha
    and the score gradient in the same kernel
    (tgx_edge_mlp_attention_backward), then sums the value gradient over the
    transposed CSR with the recomputed weights.  The reference's fused
    edge-attention keeps the same per-row state (m, l) and recomputes the
    weights in its VJP (compiler/edge_nn_attention.py:127-338, 344-611).

    Inputs after (graph, chain, roles, n_seg): value [n_src, *F], the n_seg
    field tensors, then per layer the Linear weight and bias and the
    LayerNorm weight and bias (None allowed)."""

    @staticmethod
    def forward(ctx, graph: Graph, chain, roles, n_seg: int, value: torch.Tensor, *tensors):
        _on_graph_device(graph, value, *tensors)
        segs = [_as_rows(t) for t in tensors[:n_seg]]
        params = tensors[n_seg:]
        row_ptr, col_idx = graph._kernel_csr()
        E, n_dst = col_idx.numel(), graph.schema.num_dst
        W = _padded_width(chain, sum(s.shape[1] for s in segs))
        dev = col_idx.device
        buf = torch.zeros(len(chain), _block_floats(chain, W), dtype=torch.float32, device=dev)
        _fill_weights(buf, chain, params, W, len(chain))
        mlp = _mlp_struct(chain, roles, segs, buf, W)
        stream = _native.stream_of(col_idx)
        # The scores live only for this forward; value rows of at most 8
        # floats are summed in the softmax pass itself (no per-edge weight
        # is written), wider ones by the CSR sum over the weights.
        scores = torch.empty(E, dtype=torch.float32, device=dev)
        _native.call("tgx_edge_mlp_scores", col_idx.data_ptr(), graph._dst_index32().data_ptr(),
                     _native.idx_bits(row_ptr), E, ctypes.byref(mlp), scores.data_ptr(), stream)
        lse = torch.empty(max(n_dst, 1), dtype=torch.float32, device=dev)
        out = _fused_softmax_sum(graph, scores, TGX_ROLE_EDGE, 1.0, value, lse)
        if out is not None:
            vc, F = _aligned(value), 1
            for d in value.shape[1:]:
                F *= d
        else:
            alpha = torch.empty_like(scores)
            _native.call("tgx_segment_softmax_fwd", row_ptr.data_ptr(),
                         _native.idx_bits(row_ptr), n_dst, scores.data_ptr(), alpha.data_ptr(),
                         lse.data_ptr(), stream)
            out, vc, _, F = _csr_sum_launch(value, alpha, graph)
            del alpha
        del scores
        ctx.graph, ctx.chain, ctx.roles, ctx.n_seg, ctx.W, ctx.F = graph, chain, roles, n_seg, W, F
        # A value that is also a source field of the score (the reference's
        # GAT example: value src.x, score over src.x): its two gradients meet
        # per edge in the backward kernel, so one transposed reduction
        # yields both and the value-gradient pass is skipped.
        ctx.fold = next((i for i in range(n_seg)
                         if roles[i] == "src" and tensors[i] is value
                         and segs[i].shape[1] == F), -1)
        ctx.shapes = [t.shape for t in tensors[:n_seg]]
        ctx.present = [t is not None for t in params]
        ctx.save_for_backward(buf, lse, out, vc, *segs)
        return out

    @staticmethod
    def backward(ctx, dout):
        buf, lse, out, vc, *segs = ctx.saved_tensors
        graph, chain, roles, W, F = ctx.graph, ctx.chain, ctx.roles, ctx.W, ctx.F
        row_ptr, col_idx = graph._kernel_csr()
        E, n_dst, n_src = col_idx.numel(), graph.schema.num_dst, graph.schema.num_src
        dev = col_idx.device
        L = len(chain)
        g = _aligned(dout.to(torch.float32))
        fold = ctx.fold if ctx.needs_input_grad[4] else -1
        alpha = (torch.empty(max(E, 1), dtype=torch.float32, device=dev)
                 if ctx.needs_input_grad[4] and fold < 0 else None)
        dsegs = [torch.empty(E, s.shape[1], dtype=torch.float32, device=dev) for s in segs]
        mlp = _mlp_struct(chain, roles, segs, buf, W)
        ws_bytes = ctypes.c_size_t()
        _native.call("tgx_edge_mlp_backward_workspace", E, ctypes.byref(mlp),
                     ctypes.byref(ws_bytes))
        ws = torch.empty(max(ws_bytes.value, 4), dtype=torch.uint8, device=dev)
        dweights = torch.empty(L, buf.shape[1], dtype=torch.float32, device=dev)
        ptrs = (ctypes.c_void_p * 4)(*[d.data_ptr() for d in dsegs], *([None] * (4 - len(dsegs))))
        stream = _native.stream_of(col_idx)
        _native.call("tgx_edge_mlp_attention_backward", col_idx.data_ptr(),
                     graph._dst_index32().data_ptr(), _native.idx_bits(row_ptr), E,
                     ctypes.byref(mlp), lse.data_ptr(), out.data_ptr(), g.data_ptr(),
                     vc.data_ptr(), F, _p(alpha), fold, dweights.data_ptr(), ptrs,
                     ws.data_ptr(), ws_bytes.value, stream)
        dvalue = None
        if alpha is not None:
            dvalue = torch.empty_like(vc)
            if n_src and F:
                t = graph._transposed()
                partial = _partial(t.plan, F, dev)
                _native.call("tgx_csr_sum_bwd", t.row_ptr_t.data_ptr(), t.col_t.data_ptr(),
                             t.perm.data_ptr(), t.plan.ref, vc.data_ptr(), alpha.data_ptr(),
                             g.data_ptr(), dvalue.data_ptr(), None, n_dst, n_src, F,
                             _native.DTYPE_F32, _p(partial), stream)
        # Folded: the source segment's reduction is the value's whole
        # gradient (value and field are one tensor; its gradient is returned
        # once, for the field).
        grads = _segment_grads(graph, roles, dsegs, ctx.shapes, ctx.needs_input_grad, 5)
        grads += _layer_grads(chain, dweights, W, ctx.present, ctx.needs_input_grad,
                              5 + ctx.n_seg, L)
        return (None, None, None, None, dvalue, *grads)


TGX_ROLE_SRC, TGX_ROLE_DST, TGX_ROLE_EDGE = 0, 1, 2


def _fusable(value: torch.Tensor) -> bool:
    """Value rows the one-pass softmax sum takes: fp32, 1 to 8 floats."""
    width = 1
    for d in value.shape[1:]:
        width *= d
    return value.dtype == torch.float32 and 1 <= width <= 8


def _fused_softmax_sum(graph: Graph, scores: torch.Tensor, role: int, scale: float,
                       value: torch.Tensor, lse: torch.Tensor,
                       alpha: torch.Tensor | None = None) -> torch.Tensor | None:
    """out = sum_e softmax_i(scale * score) value[col[e]] in one pass
    (tgx_segment_softmax_sum_fwd), lse (and alpha, when given) filled; None
    when the value is not fp32 rows of at most 8 floats (the caller then
    runs the softmax and the CSR sum)."""
    if not _fusable(value):
        return None
    width = 1
    for d in value.shape[1:]:
        width *= d
    row_ptr, col_idx = graph._kernel_csr()
    n_dst = graph.schema.num_dst
    vc = _aligned(value)
    out = torch.empty((n_dst, *value.shape[1:]), dtype=torch.float32, device=value.device)
    _native.call("tgx_segment_softmax_sum_fwd", row_ptr.data_ptr(), col_idx.data_ptr(),
                 _native.idx_bits(row_ptr), n_dst, scores.data_ptr(), role, float(scale),
                 vc.data_ptr(), width, _p(alpha), lse.data_ptr(), out.data_ptr(),
                 _native.stream_of(value))
    return out


def nn_attention(graph: Graph, chain, roles, fields, value: torch.Tensor) -> torch.Tensor:
    """out[i] = sum_e softmax_i(net(fields_e)) value[col[e]] on the HIP path."""
    params = _layer_params(chain)
    return NnAttentionFunction.apply(graph, chain, tuple(roles), len(fields), value, *fields,
                                     *params)


# ---------------------------------------------------------------------------
# Online softmax over a raw score field (tgx_segment_softmax_gather_fwd)

_ROLE_CODE = {"src": 0, "dst": 1, "edge": 2}


def _score_softmax_launch(table: torch.Tensor, role: str, scale: float,
                          graph: Graph) -> torch.Tensor:
    _on_graph_device(graph, table)
    row_ptr, col_idx = graph._kernel_csr()
    n = graph.schema.num_dst
    flat = table.reshape(-1).contiguous()
    alpha = torch.empty(max(col_idx.numel(), 1), dtype=torch.float32,
                        device=table.device)[:col_idx.numel()]
    lse = torch.empty(max(n, 1), dtype=torch.float32, device=table.device)
    _native.call("tgx_segment_softmax_gather_fwd", row_ptr.data_ptr(), col_idx.data_ptr(),
                 _native.idx_bits(row_ptr), n, flat.data_ptr(), _ROLE_CODE[role],
                 float(scale), alpha.data_ptr(), lse.data_ptr(), _native.stream_of(table))
    return alpha


class ScoreSoftmaxFunction(torch.autograd.Function):
    """alpha[e] = softmax over row i of scale * score(e), the score read from
    a source-node table through col[e], a destination-node table, or one
    value per edge; [E] fp32."""

    @staticmethod
    def forward(ctx, table: torch.Tensor, role: str, scale: float, graph: Graph):
        alpha = _score_softmax_launch(table, role, scale, graph)
        ctx.graph, ctx.role, ctx.scale, ctx.shape = graph, role, float(scale), table.shape
        ctx.save_for_backward(alpha)
        return alpha

    @staticmethod
    def backward(ctx, dalpha):
        (alpha,) = ctx.saved_tensors
        graph: Graph = ctx.graph
        row_ptr, _ = graph._kernel_csr()
        dalpha = dalpha.contiguous()
        dscore = torch.empty_like(alpha)
        _native.call("tgx_segment_softmax_bwd", row_ptr.data_ptr(), _native.idx_bits(row_ptr),
                     graph.schema.num_dst, alpha.data_ptr(), dalpha.data_ptr(),
                     dscore.data_ptr(), _native.stream_of(alpha))
        if ctx.role == "src":
            grad = _reduce_rows_transposed(graph, dscore[:, None])[:, 0]
        elif ctx.role == "dst":
            grad = _reduce_rows(graph, dscore[:, None])[:, 0]
        else:
            grad = dscore
        if ctx.scale != 1.0:
            grad = grad * ctx.scale
        return grad.reshape(ctx.shape), None, None, None


class ScoreAttentionFunction(torch.autograd.Function):
    """out[i] = sum_e softmax_i(scale * score(e)) value[col[e]] for fp32
    value rows of at most 8 floats: the forward is the one-pass softmax sum
    (keeping the weights for the backward), the backward the composition's:
    the value gradient over the transposed CSR with the weights, the
    weights' gradient <dout[i], value[j]> in edge order, the softmax
    Jacobian, the score gradient reduced onto the field's rows."""

    @staticmethod
    def forward(ctx, table: torch.Tensor, value: torch.Tensor, role: str, scale: float,
                graph: Graph):
        _on_graph_device(graph, table, value)
        E = graph.num_edges
        alpha = torch.empty(max(E, 1), dtype=torch.float32, device=table.device)[:E]
        lse = torch.empty(max(graph.schema.num_dst, 1), dtype=torch.float32,
                          device=table.device)
        vc = _aligned(value)
        out = _fused_softmax_sum(graph, table.reshape(-1).contiguous(), _ROLE_CODE[role],
                                 scale, vc, lse, alpha)
        ctx.graph, ctx.role, ctx.scale, ctx.shape = graph, role, float(scale), table.shape
        ctx.save_for_backward(alpha, vc)
        return out

    @staticmethod
    def backward(ctx, dout):
        alpha, vc = ctx.saved_tensors
        graph: Graph = ctx.graph
        n_dst, n_src, E = graph.schema.num_dst, graph.schema.num_src, graph.num_edges
        F = 1
        for d in vc.shape[1:]:
            F *= d
        dout = _aligned(dout.to(torch.float32))
        stream = _native.stream_of(vc)
        dvalue = dtable = None
        if ctx.needs_input_grad[1]:
            dvalue = torch.empty_like(vc)
            if n_src:
                t = graph._transposed()
                partial = _partial(t.plan, F, vc.device)
                _native.call("tgx_csr_sum_bwd", t.row_ptr_t.data_ptr(), t.col_t.data_ptr(),
                             t.perm.data_ptr(), t.plan.ref, vc.data_ptr(), alpha.data_ptr(),
                             dout.data_ptr(), dvalue.data_ptr(), None, n_dst, n_src, F,
                             _native.DTYPE_F32, _p(partial), stream)
        if ctx.needs_input_grad[0]:
            row_ptr, col_idx = graph._kernel_csr()
            dalpha = torch.empty(max(E, 1), dtype=torch.float32, device=vc.device)[:E]
            dscore = torch.empty_like(dalpha)
            if E:
                _native.call("tgx_csr_edge_dot", row_ptr.data_ptr(), col_idx.data_ptr(),
                             _native.idx_bits(row_ptr), graph._row_plan().ref, vc.data_ptr(),
                             dout.data_ptr(), dalpha.data_ptr(), n_dst, n_src, F,
                             _native.DTYPE_F32, stream)
                _native.call("tgx_segment_softmax_bwd", row_ptr.data_ptr(),
                             _native.idx_bits(row_ptr), n_dst, alpha.data_ptr(),
                             dalpha.data_ptr(), dscore.data_ptr(), stream)
            if ctx.role == "src":
                grad = _reduce_rows_transposed(graph, dscore[:, None])[:, 0]
            elif ctx.role == "dst":
                grad = _reduce_rows(graph, dscore[:, None])[:, 0]
            else:
                grad = dscore
            if ctx.scale != 1.0:
                grad = grad * ctx.scale
            dtable = grad.reshape(ctx.shape)
        return dtable, dvalue, None, None, None


def score_attention(graph: Graph, table: torch.Tensor, role: str, scale: float,
                    value: torch.Tensor) -> torch.Tensor:
    """out[i] = sum_e softmax_i(scale * score(e)) value[col[e]] on the HIP path:
    one pass (softmax and value sum) for fp32 value rows of at most 8
    floats, else the gathered segment softmax, then the weighted CSR sum.  A
    16-bit score
    field is widened to fp32 first (the softmax runs in fp32, as the
    reference's oracle accumulates); the output has the value's type."""
    if table.dtype != torch.float32:
        table = table.float()
    tracked = torch.is_grad_enabled() and (table.requires_grad or value.requires_grad)
    if _fusable(value):
        if tracked:
            return ScoreAttentionFunction.apply(table, value, role, scale, graph)
        _on_graph_device(graph, table, value)
        lse = torch.empty(max(graph.schema.num_dst, 1), dtype=torch.float32,
                          device=table.device)
        return _fused_softmax_sum(graph, table.reshape(-1).contiguous(), _ROLE_CODE[role],
                                  scale, value, lse)
    if tracked:
        alpha = ScoreSoftmaxFunction.apply(table, role, scale, graph)
    else:
        alpha = _score_softmax_launch(table, role, scale, graph)
    return csr_sum(value, alpha, graph)


# ---------------------------------------------------------------------------
# Edge-network messages summed per row (tg.sum() over tg.nn.trace(net)(...))

def _row_degrees(graph: Graph) -> torch.Tensor:
    row_ptr, _ = graph._kernel_csr()
    got = graph._native_cache.get("degree_f32")
    if got is None:
        got = (row_ptr[1:] - row_ptr[:-1]).to(torch.float32)
        graph._native_cache["degree_f32"] = got
    return got


class EdgeMlpSumFunction(torch.autograd.Function):
    """out[i] = sum over row i's edges of net(concat of the fields gathered
    for the edge).  The last Linear layer is linear, so the kernels evaluate
    the layers before it per edge (tgx_edge_mlp_hidden), the CSR sum adds
    those per row, and the last layer acts once per row:
    out = S W'^T + deg b' (W', b' its folded weights).  Backward: the
    last layer's gradients from S, and the gradient at its input,
    dS = dout W', seeds the per-edge backward of the other layers
    (tgx_edge_mlp_backward_seeded).

    Inputs after (graph, chain, roles, n_seg): the n_seg field tensors, then
    per layer the Linear weight and bias and the LayerNorm weight and bias
    (None allowed; the last layer has no LayerNorm)."""

    @staticmethod
    def forward(ctx, graph: Graph, chain, roles, n_seg: int, *tensors):
        _on_graph_device(graph, *tensors)
        segs = [_as_rows(t) for t in tensors[:n_seg]]
        params = tensors[n_seg:]
        row_ptr, col_idx = graph._kernel_csr()
        E, L = col_idx.numel(), len(chain)
        dev = col_idx.device
        in_width = sum(x.shape[1] for x in segs)
        W = _padded_width(chain, in_width, vector=True)
        hw = chain[-1].linear.in_features
        buf = torch.zeros(L, _block_floats(chain, W), dtype=torch.float32, device=dev)
        _fill_weights(buf, chain, params, W, L - 1)
        mlp = _mlp_struct(chain, roles, segs, buf, W)
        hidden = torch.empty(max(E, 1), hw, dtype=torch.float32, device=dev)[:E]
        _native.call("tgx_edge_mlp_hidden", col_idx.data_ptr(), graph._dst_index32().data_ptr(),
                     _native.idx_bits(row_ptr), E, ctypes.byref(mlp), hidden.data_ptr(), hw,
                     _native.stream_of(col_idx))
        sums = _reduce_rows(graph, hidden)
        w_last, b_last = _folded(chain[-1], params[_PER_LAYER * (L - 1)],
                                 params[_PER_LAYER * (L - 1) + 1])
        out = sums @ w_last.t()
        if b_last is not None:
            out = out + _row_degrees(graph)[:, None] * b_last
        ctx.graph, ctx.chain, ctx.roles, ctx.n_seg, ctx.W = graph, chain, roles, n_seg, W
        ctx.shapes = [t.shape for t in tensors[:n_seg]]
        ctx.present = [t is not None for t in params]
        ctx.save_for_backward(buf, sums, w_last, *segs)
        return out

    @staticmethod
    def backward(ctx, dout):
        buf, sums, w_last, *segs = ctx.saved_tensors
        graph, chain, roles, W = ctx.graph, ctx.chain, ctx.roles, ctx.W
        row_ptr, col_idx = graph._kernel_csr()
        E, L = col_idx.numel(), len(chain)
        dev = col_idx.device
        dout = dout.contiguous()
        needs = ctx.needs_input_grad
        last = chain[-1]
        k_last = 4 + ctx.n_seg + _PER_LAYER * (L - 1)
        need_w = needs[k_last]
        need_b = ctx.present[_PER_LAYER * (L - 1) + 1] and needs[k_last + 1]
        dwf = (dout.t() @ sums) if need_w else None
        dbf = (_row_degrees(graph)[:, None] * dout).sum(0) \
            if need_b or (need_w and last.in_shift != 0.0) else None
        d_w_last, d_b_last = _unfolded_grads(last, dwf, dbf, need_w, need_b)
        grads = [None] * ctx.n_seg
        grads += [None] * (_PER_LAYER * (L - 1))
        upstream = any(needs[4:k_last])
        if upstream:
            seed = (dout @ w_last).contiguous()
            hw = seed.shape[1]
            dsegs = [torch.empty(max(E, 1), x.shape[1], dtype=torch.float32,
                                 device=dev)[:E] for x in segs]
            mlp = _mlp_struct(chain, roles, segs, buf, W)
            ws_bytes = ctypes.c_size_t()
            _native.call("tgx_edge_mlp_backward_workspace", E, ctypes.byref(mlp),
                         ctypes.byref(ws_bytes))
            ws = torch.empty(max(ws_bytes.value, 4), dtype=torch.uint8, device=dev)
            dweights = torch.empty(L, buf.shape[1], dtype=torch.float32, device=dev)
            ptrs = (ctypes.c_void_p * 4)(*[d.data_ptr() for d in dsegs],
                                         *([None] * (4 - len(dsegs))))
            _native.call("tgx_edge_mlp_backward_seeded", col_idx.data_ptr(),
                         graph._dst_index32().data_ptr(), _native.idx_bits(row_ptr), E,
                         ctypes.byref(mlp), seed.data_ptr(), hw, dweights.data_ptr(), ptrs,
                         ws.data_ptr(), ws_bytes.value, _native.stream_of(col_idx))
            grads = _segment_grads(graph, roles, dsegs, ctx.shapes, needs, 4)
            grads += _layer_grads(chain, dweights, W, ctx.present, needs, 4 + ctx.n_seg, L - 1)
        return (None, None, None, None, *grads, d_w_last, d_b_last, None, None)


def nn_message_sum(graph: Graph, chain, roles, fields) -> torch.Tensor:
    """out[i] = sum_e net(fields_e) over row i's edges on the HIP path."""
    params = _layer_params(chain)
    return EdgeMlpSumFunction.apply(graph, chain, tuple(roles), len(fields), *fields, *params)

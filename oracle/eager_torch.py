"""The reference's CPU path for Torch tensors, restated with Torch CPU ops.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py): timed by bench.py as the
CPU baseline, never used by the product.

For Torch inputs on a general CSR the reference runs its eager oracle:
``_evaluate_reference`` gathers src[col] and dst[destination] per edge, runs
the user's edge() in Torch, then ``reduce_online_softmax``
(scatter_reduce amax -> exp -> index_add x2 -> guarded divide) or
``reduce_sum`` (index_add), and Torch autograd supplies the backward
(python/tiga/interop/torch/message_passing.py:2848-2894,
python/tiga/interop/torch/reducer_oracle.py:44-137).  The weighted sum on CPU
dispatches torch.sparse.mm (message_passing.py:3284-3345).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def destination_index(row_ptr: torch.Tensor) -> torch.Tensor:
    degree = row_ptr[1:] - row_ptr[:-1]
    return torch.repeat_interleave(torch.arange(row_ptr.numel() - 1), degree)


def reduce_online_softmax(score, value, destination, num_dst):
    acc = torch.float32 if score.dtype in (torch.float16, torch.bfloat16) else score.dtype
    score_acc = score.to(acc)
    value_acc = value.to(acc)
    lanes = tuple(score.shape[1:])
    payload_rank = value.ndim - score.ndim
    maximum = torch.full((num_dst, *lanes), -torch.inf, dtype=acc)
    index = destination.reshape(-1, *((1,) * len(lanes))).expand_as(score_acc)
    maximum = maximum.scatter_reduce(0, index, score_acc, reduce="amax", include_self=True)
    scale = torch.exp(score_acc - maximum[destination])
    denominator = torch.zeros_like(maximum).index_add(0, destination, scale)
    value_scale = scale.reshape(*scale.shape, *((1,) * payload_rank))
    numerator = torch.zeros((num_dst, *value.shape[1:]), dtype=acc).index_add(
        0, destination, value_acc * value_scale)
    denominator = denominator.reshape(*denominator.shape, *((1,) * payload_rank))
    out = torch.where(denominator > 0,
                      numerator / denominator.clamp_min(torch.finfo(acc).tiny),
                      torch.zeros_like(numerator))
    return out.to(value.dtype)


def gat_step(row_ptr, col, h, a_src, a_dst, slope, dout):
    """One GAT forward + backward on the eager path (CPU tensors)."""
    destination = destination_index(row_ptr)
    num_dst = row_ptr.numel() - 1
    h = h.detach().requires_grad_(True)
    a_src = a_src.detach().requires_grad_(True)
    a_dst = a_dst.detach().requires_grad_(True)
    hs = h[col]
    hd = h[destination]
    score = F.leaky_relu((hs * a_src).sum(-1) + (hd * a_dst).sum(-1), slope)
    out = reduce_online_softmax(score, hs, destination, num_dst)
    out.backward(dout)
    return out, h.grad, a_src.grad, a_dst.grad


def dot_step(row_ptr, col, q, k, v, bias, scale, dout=None):
    """Dot-product attention forward (+ backward when dout is given)."""
    destination = destination_index(row_ptr)
    num_dst = row_ptr.numel() - 1
    leaves = [t.detach().requires_grad_(dout is not None) for t in (q, k, v, bias)]
    q, k, v, bias = leaves
    score = (k[col] * q[destination]).sum(dim=-1) * scale + bias
    out = reduce_online_softmax(score, v[col], destination, num_dst)
    if dout is not None:
        out.backward(dout)
    return out


def sum_step(row_ptr, col, x, w, dout):
    """Weighted sum via torch.sparse.mm forward + autograd backward."""
    destination = destination_index(row_ptr)
    n_dst = row_ptr.numel() - 1
    x = x.detach().requires_grad_(True)
    w = w.detach().requires_grad_(True)
    a = torch.sparse_coo_tensor(torch.stack([destination, col]), w, (n_dst, x.shape[0]))
    out = torch.sparse.mm(a, x)
    out.backward(dout)
    return out, x.grad, w.grad


def nn_gat_step(row_ptr, col, x, disp, net, dout):
    """The nn-scored GAT step on the eager path (CPU tensors): score =
    net(cat[displacement, x_src, x_dst]) per edge (a tg.nn.trace module
    applied to its concatenated inputs, compiler/nn_capture.py:1-33), online
    softmax over each destination row, value x_src; forward + backward into
    x, the displacement and the network's parameters."""
    destination = destination_index(row_ptr)
    num_dst = row_ptr.numel() - 1
    x = x.detach().requires_grad_(True)
    disp = disp.detach().requires_grad_(True)
    score = net(torch.cat([disp, x[col], x[destination]], dim=1))[:, 0]
    out = reduce_online_softmax(score, x[col], destination, num_dst)
    out.backward(dout)
    return out, x.grad, disp.grad


def dot_reference(row_ptr, col, q, k, v, bias, scale, dout):
    """The reference's eager arithmetic for dot-product attention, forward
    and backward, in the inputs' own dtypes: for bf16 q/k/v the products
    k[col] * q[dst] and their sum over D are bf16 (Torch's bf16 ops), the
    fp32 bias promotes the score to fp32, reduce_online_softmax accumulates
    in fp32 and casts the output back to bf16 (reducer_oracle.py:22-41, 87-91,
    137); Torch autograd gives the gradients.  Returns (out, dq, dk, dv,
    dbias) (dbias None without a bias)."""
    destination = destination_index(row_ptr)
    num_dst = row_ptr.numel() - 1
    q, k, v = (t.detach().requires_grad_(True) for t in (q, k, v))
    b = None if bias is None else bias.detach().requires_grad_(True)
    score = (k[col] * q[destination]).sum(dim=-1) * scale
    if b is not None:
        score = score + b
    out = reduce_online_softmax(score, v[col], destination, num_dst)
    out.backward(dout)
    return out.detach(), q.grad, k.grad, v.grad, None if b is None else b.grad


def _gathered(row_ptr, col, inputs):
    """Feature-concatenation of the fields gathered per edge, and the leaves
    (inputs = [(role, tensor [rows] or [rows, k])])."""
    destination = destination_index(row_ptr)
    leaves, parts = [], []
    for role, t in inputs:
        leaf = t.detach().requires_grad_(True)
        leaves.append(leaf)
        x = leaf if leaf.ndim == 2 else leaf[:, None]
        parts.append(x[col] if role == "src" else x[destination] if role == "dst" else x)
    return torch.cat(parts, dim=1), destination, leaves


def nn_message_sum(row_ptr, col, inputs, net, dout):
    """The eager path of tg.sum() over tg.nn.trace(net)(fields...): the
    module on the concatenated gathered fields, index_add per destination
    row (reduce_sum, reducer_oracle.py:44-57), Torch autograd.  Runs in the
    inputs' dtype (float64 for checking).  Returns (out, input grads,
    parameter grads in net.parameters() order)."""
    x, destination, leaves = _gathered(row_ptr, col, inputs)
    msg = net(x)
    out = torch.zeros(row_ptr.numel() - 1, msg.shape[1], dtype=msg.dtype).index_add(
        0, destination, msg)
    params = [p for p in net.parameters()]
    grads = torch.autograd.grad(out, leaves + params, dout, allow_unused=True)
    return out.detach(), list(grads[:len(leaves)]), list(grads[len(leaves):])


def nn_attention(row_ptr, col, inputs, net, value, dout, out_scale=1.0):
    """The eager path of online_softmax(score = out_scale * net(fields...),
    value = src.value) with Torch autograd (reducer_oracle.py:60-137).
    Returns (out, input grads, value grad, parameter grads)."""
    x, destination, leaves = _gathered(row_ptr, col, inputs)
    v = value.detach().requires_grad_(True)
    score = net(x)[:, 0] * out_scale
    out = reduce_online_softmax(score, v[col], destination, row_ptr.numel() - 1)
    params = [p for p in net.parameters()]
    grads = torch.autograd.grad(out, leaves + [v] + params, dout, allow_unused=True)
    n = len(leaves)
    return out.detach(), list(grads[:n]), grads[n], list(grads[n + 1:])

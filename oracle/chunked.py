"""Row-chunked float64 restatement of the GAT and dot-product attention
passes, of per-sequence causal attention and of nn-scored attention, for
checking full-size outputs.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py): never imported by the
product.

The arithmetic is ``ref.gat_fwd/gat_bwd`` and ``ref.dot_fwd/dot_bwd`` (the
reference's ``_evaluate_reference`` + ``reduce_online_softmax``,
python/tiga/interop/torch/message_passing.py:2848-2894 and
python/tiga/interop/torch/reducer_oracle.py:60-137, differentiated as its
Torch autograd would), in float64, but over contiguous blocks of destination
rows so that the per-edge gathers of a 17M- or 32M-edge graph never exist at
once.  Written with Torch ops on whatever device the inputs are on: pinned
against ``ref`` on small graphs on the CPU (tests/test_oracle.py); the
full-size GPU tests run it in float64 on the GPU, where Torch's own kernels,
not libtgx_hip.so, compute it.

Every function takes int64 ``row_ptr``/``col`` and float64 node tensors and
returns float64 results.
"""

from __future__ import annotations

import torch


def row_blocks(row_ptr: torch.Tensor, edges_per_block: int):
    """Contiguous destination-row ranges [r0, r1) of about
    `edges_per_block` edges each (a row is never split)."""
    rp = row_ptr.to("cpu", torch.int64)
    n = rp.numel() - 1
    r0 = 0
    while r0 < n:
        target = int(rp[r0]) + edges_per_block
        r1 = int(torch.searchsorted(rp, target, right=True)) - 1
        r1 = min(max(r1, r0 + 1), n)
        yield r0, r1
        r0 = r1


def _block(row_ptr, col, r0, r1):
    """(e0, e1, local destination of each edge, source of each edge)."""
    e0, e1 = int(row_ptr[r0]), int(row_ptr[r1])
    degree = row_ptr[r0 + 1:r1 + 1] - row_ptr[r0:r1]
    local = torch.repeat_interleave(torch.arange(r1 - r0, device=col.device), degree)
    return e0, e1, local, col[e0:e1]


def _segment_softmax(score, value, local, rows):
    """(out, lse, alpha) of one row block: score [e, H], value [e, H, D]."""
    H = score.shape[1]
    m = torch.full((rows, H), -torch.inf, dtype=score.dtype, device=score.device)
    m = m.scatter_reduce(0, local[:, None].expand_as(score), score, "amax", include_self=True)
    p = torch.exp(score - m[local])
    den = torch.zeros_like(m).index_add_(0, local, p)
    num = torch.zeros((rows, *value.shape[1:]), dtype=value.dtype, device=value.device)
    num.index_add_(0, local, p[..., None] * value)
    safe = torch.where(den > 0, den, torch.ones_like(den))
    out = torch.where(den[..., None] > 0, num / safe[..., None], torch.zeros_like(num))
    lse = torch.where(den > 0, m + torch.log(safe), torch.full_like(m, -torch.inf))
    alpha = p / safe[local]
    return out, lse, alpha


def _leaky(z, slope):
    return torch.where(z > 0, z, z * slope)


def gat_fwd(row_ptr, col, h, a_src, a_dst, slope, edges_per_block=1 << 19):
    """GAT forward: (out [N, H, D], lse [N, H]) as ref.gat_fwd."""
    n = row_ptr.numel() - 1
    ss = (h * a_src).sum(-1)
    sd = (h * a_dst).sum(-1)
    out = torch.zeros((n, *h.shape[1:]), dtype=h.dtype, device=h.device)
    lse = torch.full((n, h.shape[1]), -torch.inf, dtype=h.dtype, device=h.device)
    for r0, r1 in row_blocks(row_ptr, edges_per_block):
        e0, e1, local, src = _block(row_ptr, col, r0, r1)
        if e1 == e0:
            continue
        s = _leaky(ss[src] + sd[r0 + local], slope)
        o, l, _ = _segment_softmax(s, h[src], local, r1 - r0)
        out[r0:r1] = o
        lse[r0:r1] = l
    return out, lse


def gat_bwd(row_ptr, col, h, a_src, a_dst, slope, dout, edges_per_block=1 << 19,
            branch=None, stats=None):
    """(dh, da_src, da_dst) as ref.gat_bwd: the softmax adjoint per edge,
    LeakyReLU'(0) = slope, source-side terms added at col, destination-side
    terms at the row.

    LeakyReLU's derivative jumps at z = 0.  `branch`, optional, is a pair
    (zs [N, H], zd [N, H]) of the checked implementation's own fp32 source
    and destination halves of z: the derivative's piece is then chosen by
    the sign of zs[j] + zd[i] (one fp32 addition, as that implementation
    forms it), so that both differentiate the same piece of the function
    where fp32 and fp64 values of z straddle 0.  `stats`, a dict, receives
    the number of (edge, head) pairs whose two signs differ."""
    ss = (h * a_src).sum(-1)
    sd = (h * a_dst).sum(-1)
    dh = torch.zeros_like(h)
    da_src = torch.zeros_like(a_src)
    da_dst = torch.zeros_like(a_dst)
    flips = 0
    for r0, r1 in row_blocks(row_ptr, edges_per_block):
        e0, e1, local, src = _block(row_ptr, col, r0, r1)
        if e1 == e0:
            continue
        dst = r0 + local
        z = ss[src] + sd[dst]
        value = h[src]
        out, _, alpha = _segment_softmax(_leaky(z, slope), value, local, r1 - r0)
        g = dout[dst]
        delta = (dout[r0:r1] * out).sum(-1)
        dscore = alpha * ((g * value).sum(-1) - delta[local])
        positive = z > 0
        if branch is not None:
            kernel_positive = (branch[0][src] + branch[1][dst]) > 0
            flips += int((kernel_positive != positive).sum())
            positive = kernel_positive
        dz = torch.where(positive, dscore, dscore * slope)
        dh.index_add_(0, src, alpha[..., None] * g + dz[..., None] * a_src)
        dh.index_add_(0, dst, dz[..., None] * a_dst)
        da_src += (dz[..., None] * value).sum(0)
        da_dst += (dz[..., None] * h[dst]).sum(0)
    if stats is not None:
        stats["kink_flips"] = flips
    return dh, da_src, da_dst


def dot_fwd(row_ptr, col, q, k, v, scale, bias=None, rows=None, edges_per_block=1 << 19):
    """Dot-product attention forward (out [N, H, D], lse [N, H]) as
    ref.dot_fwd.  `rows` (optional, sorted int64 on the CPU) restricts the
    evaluation to those destination rows; other rows stay 0 / -inf."""
    n = row_ptr.numel() - 1
    out = torch.zeros((n, *q.shape[1:]), dtype=q.dtype, device=q.device)
    lse = torch.full((n, q.shape[1]), -torch.inf, dtype=q.dtype, device=q.device)
    ranges = row_blocks(row_ptr, edges_per_block) if rows is None else \
        ((int(r), int(r) + 1) for r in rows)
    for r0, r1 in ranges:
        e0, e1, local, src = _block(row_ptr, col, r0, r1)
        if e1 == e0:
            continue
        s = (k[src] * q[r0 + local]).sum(-1) * scale
        if bias is not None:
            s = s + bias[e0:e1]
        o, l, _ = _segment_softmax(s, v[src], local, r1 - r0)
        out[r0:r1] = o
        lse[r0:r1] = l
    return out, lse


def dot_bwd(row_ptr, col, q, k, v, scale, bias, dout, edges_per_block=1 << 19):
    """(dq, dk, dv, dbias) as ref.dot_bwd (dbias = the score gradient per
    edge, [E, H])."""
    dq = torch.zeros_like(q)
    dk = torch.zeros_like(k)
    dv = torch.zeros_like(v)
    dbias = torch.zeros((col.numel(), q.shape[1]), dtype=q.dtype, device=q.device)
    for r0, r1 in row_blocks(row_ptr, edges_per_block):
        e0, e1, local, src = _block(row_ptr, col, r0, r1)
        if e1 == e0:
            continue
        dst = r0 + local
        ks, vs, qd = k[src], v[src], q[dst]
        s = (ks * qd).sum(-1) * scale
        if bias is not None:
            s = s + bias[e0:e1]
        out, _, alpha = _segment_softmax(s, vs, local, r1 - r0)
        g = dout[dst]
        delta = (dout[r0:r1] * out).sum(-1)
        dscore = alpha * ((g * vs).sum(-1) - delta[local])
        dbias[e0:e1] = dscore
        dq.index_add_(0, dst, dscore[..., None] * ks * scale)
        dk.index_add_(0, src, dscore[..., None] * qd * scale)
        dv.index_add_(0, src, alpha[..., None] * g)
    return dq, dk, dv, dbias


def causal_sequence(q, k, v, scale, dout=None, query_block=512):
    """One sequence of causal softmax attention, float64, over blocks of
    query rows: (out [L, H, D], lse [L, H]) and, with `dout`, also
    (dq, dk, dv).  The arithmetic of ``ref.varlen_causal_fwd/bwd`` (the
    dot-product relation on Graph.cu_seqlens(causal=True); per-sequence
    causal SDPA as the reference's tests/python/test_attention_examples.py:
    53-72 checks it) with the score matrix formed `query_block` rows at a
    time, so a 4096-token, 16-head sequence needs about 270 MB at once.

    The backward's row term is delta_i = <dout_i, out_i> from the float64
    output; probabilities are recomputed from the saved logsumexp."""
    L, H, D = q.shape
    qh, kh, vh = (t.permute(1, 0, 2).contiguous() for t in (q, k, v))     # [H, L, D]
    out = torch.empty((H, L, D), dtype=q.dtype, device=q.device)
    lse = torch.empty((H, L), dtype=q.dtype, device=q.device)
    keys = torch.arange(L, device=q.device)

    def probabilities(i0, i1):
        s = torch.matmul(qh[:, i0:i1], kh[:, :i1].transpose(1, 2).contiguous()) * scale
        mask = keys[None, :i1] <= torch.arange(i0, i1, device=q.device)[:, None]
        return s.masked_fill(~mask[None], -torch.inf)

    for i0 in range(0, L, query_block):
        i1 = min(i0 + query_block, L)
        s = probabilities(i0, i1)
        m = s.amax(-1, keepdim=True)
        p = torch.exp(s - m)
        den = p.sum(-1, keepdim=True)
        out[:, i0:i1] = torch.matmul(p / den, vh[:, :i1])
        lse[:, i0:i1] = (m + torch.log(den))[..., 0]
    if dout is None:
        return out.permute(1, 0, 2), lse.T
    gh = dout.permute(1, 0, 2).contiguous()
    delta = (gh * out).sum(-1)                                              # [H, L]
    dq = torch.empty_like(qh)
    dk = torch.zeros_like(kh)
    dv = torch.zeros_like(vh)
    for i0 in range(0, L, query_block):
        i1 = min(i0 + query_block, L)
        p = torch.exp(probabilities(i0, i1) - lse[:, i0:i1, None])          # [H, b, i1]
        dp = torch.matmul(gh[:, i0:i1], vh[:, :i1].transpose(1, 2).contiguous())
        ds = p * (dp - delta[:, i0:i1, None])
        dq[:, i0:i1] = torch.matmul(ds, kh[:, :i1]) * scale
        dk[:, :i1] += torch.matmul(ds.transpose(1, 2).contiguous(), qh[:, i0:i1]) * scale
        dv[:, :i1] += torch.matmul(p.transpose(1, 2).contiguous(), gh[:, i0:i1])
    back = lambda t: t.permute(1, 0, 2)
    return back(out), lse.T, back(dq), back(dk), back(dv)


def _activate(name, z, p):
    """ref._act in Torch ops (the same closed forms)."""
    if name == "relu":
        return torch.clamp_min(z, 0.0)
    if name == "leaky_relu":
        return torch.where(z > 0, z, p * z)
    if name == "tanh":
        return torch.tanh(z)
    if name == "sigmoid":
        return torch.sigmoid(z)
    if name == "silu":
        return z * torch.sigmoid(z)
    if name == "gelu":
        return 0.5 * z * (1.0 + torch.erf(z / 2.0 ** 0.5))
    if name == "elu":
        return torch.where(z > 0, z, p * torch.expm1(torch.clamp_max(z, 0.0)))
    return z


def nn_attention(row_ptr, col, inputs, layers, value, dout, keep_hidden=False):
    """``ref.nn_attention_fwd/bwd`` in float64 Torch ops with autograd (the
    whole graph at once: a 4M-edge relation's [E, 19] float64 gathers fit
    on the GPU).  inputs = [(role, [rows, w])], layers = [(W, b or None,
    act, param)] as float64 tensors.  The row maximum is held constant,
    which softmax shift-invariance makes exact.  Returns (out, [d inputs],
    d value, [(dW, db or None)]), and with keep_hidden a fifth item: per
    hidden layer (input a [E, in], pre-activation z [E, out], dz [E, out])."""
    n = row_ptr.numel() - 1
    dst = torch.repeat_interleave(torch.arange(n, device=col.device),
                                  row_ptr[1:] - row_ptr[:-1])
    leaves = [t.detach().clone().requires_grad_(True) for _, t in inputs]
    parts = [t[col] if role == "src" else t[dst] if role == "dst" else t
             for (role, _), t in zip(inputs, leaves)]
    a = torch.cat(parts, dim=1)
    params, hidden = [], []
    for i, (W, b, act, p) in enumerate(layers):
        Wl = W.detach().clone().requires_grad_(True)
        bl = None if b is None else b.detach().clone().requires_grad_(True)
        params.append((Wl, bl))
        z = a @ Wl.T + (0.0 if bl is None else bl)
        if i + 1 < len(layers):
            hidden.append((a, z))
            a = _activate(act, z, p)
        else:
            a = z
    s = a[:, 0]
    v = value.detach().clone().requires_grad_(True)
    m = torch.full((n,), -torch.inf, dtype=s.dtype, device=s.device)
    m = m.scatter_reduce(0, dst, s.detach(), "amax", include_self=True)
    p_e = torch.exp(s - m[dst])
    den = torch.zeros(n, dtype=s.dtype, device=s.device).index_add(0, dst, p_e)
    num = torch.zeros((n, v.shape[1]), dtype=s.dtype, device=s.device)
    num = num.index_add(0, dst, v[col] * p_e[:, None])
    safe = torch.where(den > 0, den, torch.ones_like(den))
    out = torch.where(den[:, None] > 0, num / safe[:, None], torch.zeros_like(num))
    wanted = leaves + [v] + [t for pair in params for t in pair if t is not None]
    if keep_hidden:
        wanted += [z for _, z in hidden]
    grads = torch.autograd.grad(out, wanted, dout)
    k = len(leaves)
    d_inputs, d_value, rest = list(grads[:k]), grads[k], list(grads[k + 1:])
    d_layers = []
    for Wl, bl in params:
        dW = rest.pop(0)
        d_layers.append((dW, rest.pop(0) if bl is not None else None))
    if not keep_hidden:
        return out.detach(), d_inputs, d_value, d_layers
    kept = [(a_l.detach(), z.detach(), dz) for (a_l, z), dz in zip(hidden, rest)]
    return out.detach(), d_inputs, d_value, d_layers, kept

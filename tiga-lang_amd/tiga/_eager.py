"""Eager Torch evaluation for edge functions no HIP kernel covers.

Restates the reference's own fallback: gather fields per edge, run the user's
``edge()`` on Torch tensors, reduce per destination
(python/tiga/interop/torch/message_passing.py:2848-2894 and
python/tiga/interop/torch/reducer_oracle.py:44-137).  Differentiable through
Torch autograd.  Used for generic edge functions and CPU tensors only; the
recognized hot-path patterns never route here on a GPU.
"""

from __future__ import annotations

from types import SimpleNamespace

import torch

from .reducer import OnlineSoftmaxItem, OnlineSoftmaxReducer, ReducerCall, SumReducer


def _accumulation_dtype(reducer: OnlineSoftmaxReducer, score: torch.Tensor) -> torch.dtype:
    dtype = reducer.accumulation_dtype
    if dtype is None:
        return torch.float32 if score.dtype in (torch.float16, torch.bfloat16) else score.dtype
    if isinstance(dtype, torch.dtype):
        return dtype
    mapping = {"float32": torch.float32, "float64": torch.float64}
    name = getattr(dtype, "name", dtype)
    if name not in mapping:
        raise TypeError("online_softmax accumulation_dtype must be a floating dtype")
    return mapping[name]


def reduce_sum(reducer: SumReducer, message, destination, num_dst):
    out = torch.full((num_dst, *message.shape[1:]), reducer.identity(), dtype=message.dtype,
                     device=message.device)
    return out.index_add(0, destination, message)


def reduce_online_softmax(reducer: OnlineSoftmaxReducer, item: OnlineSoftmaxItem,
                          destination, num_dst):
    score, value = item.score, item.value
    if not isinstance(score, torch.Tensor) or not isinstance(value, torch.Tensor):
        raise TypeError("online_softmax score and value must be Tensors")
    while score.ndim > 1 and score.shape[-1] == 1:
        score = score.squeeze(-1)
    if score.ndim < 1 or value.ndim < score.ndim:
        raise ValueError("online_softmax requires score [edges, *lanes] and value "
                         "[edges, *lanes, *payload]")
    if score.shape[0] != destination.numel() or value.shape[0] != score.shape[0]:
        raise ValueError("online_softmax score/value leading dimension must be edges")
    if tuple(value.shape[1:score.ndim]) != tuple(score.shape[1:]):
        raise ValueError("online_softmax value must begin with the score lane dimensions")
    if not score.is_floating_point() or not value.is_floating_point():
        raise TypeError("online_softmax score and value must be floating point")
    acc = _accumulation_dtype(reducer, score)
    score_acc = score.to(acc)
    value_acc = value.to(acc)
    lanes = tuple(score.shape[1:])
    payload_rank = value.ndim - score.ndim
    maximum = torch.full((num_dst, *lanes), -torch.inf, device=score.device, dtype=acc)
    index = destination.reshape(destination.shape[0], *((1,) * len(lanes))).expand_as(score_acc)
    maximum = maximum.scatter_reduce(0, index, score_acc, reduce="amax", include_self=True)
    scale = torch.exp(score_acc - maximum[destination])
    denominator = torch.zeros_like(maximum).index_add(0, destination, scale)
    value_scale = scale.reshape(*scale.shape, *((1,) * payload_rank))
    numerator = torch.zeros((num_dst, *value.shape[1:]), device=value.device,
                            dtype=acc).index_add(0, destination, value_acc * value_scale)
    denominator = denominator.reshape(*denominator.shape, *((1,) * payload_rank))
    result = torch.where(denominator > 0,
                         numerator / denominator.clamp_min(torch.finfo(acc).tiny),
                         torch.zeros_like(numerator))
    return result.to(value.dtype)


def evaluate(kernel, graph, src, dst, edge, params):
    from .message_passing import _call_region

    row_ptr, col_idx = graph.resolve_csr()
    destination = graph.destination_index(row_ptr)
    src_at_edge = SimpleNamespace(**{n: v[col_idx] for n, v in src.items()})
    dst_at_edge = SimpleNamespace(**{n: v[destination] for n, v in dst.items()})
    message = _call_region(kernel.edge, (src_at_edge, dst_at_edge, SimpleNamespace(**edge)),
                           params)
    num_dst = graph.schema.num_dst
    if isinstance(kernel.reducer, OnlineSoftmaxReducer):
        if not isinstance(message, OnlineSoftmaxItem):
            raise TypeError("online_softmax edge() must return self.reducer(score, value)")
        return reduce_online_softmax(kernel.reducer, message, destination, num_dst)
    if isinstance(message, ReducerCall):
        if len(message.messages) != 1:
            raise NotImplementedError("multi-message reducer bindings are not supported")
        message = message.messages[0]
    if isinstance(kernel.reducer, SumReducer):
        return reduce_sum(kernel.reducer, message, destination, num_dst)
    raise NotImplementedError(f"no evaluator for reducer {type(kernel.reducer).__name__}")

"""Reducers accepted by :class:`tiga.MessagePassing`.

Same public surface as the reference's ``python/tiga/reducer/core.py``
(``Reducer`` 24-87, ``SumReducer`` 90-109, ``OnlineSoftmaxItem`` 112-117,
``OnlineSoftmaxReducer`` 160-202, factories 205-229): a reducer is a small
algebra object; ``edge()`` returns either a message tensor (sum) or
``self.reducer(score, value)`` (online softmax).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any


@dataclass(frozen=True)
class ReducerCall:
    """What ``reducer(*messages)`` returns inside ``edge()``: the reducer and
    the per-edge message expressions it will reduce."""

    reducer: "Reducer"
    messages: tuple[Any, ...]


@dataclass(frozen=True)
class OnlineSoftmaxItem:
    """What ``online_softmax()(score, value)`` returns inside ``edge()``: the
    per-edge score [E, *lanes] and value [E, *lanes, *payload] to reduce."""

    score: Any
    value: Any


class Reducer:
    name = "custom"
    associative = False
    commutative = False

    def __init__(self, *, deterministic: bool = False) -> None:
        self.deterministic = bool(deterministic)

    def identity(self):
        raise NotImplementedError

    def combine(self, left, right):
        raise NotImplementedError

    def finalize(self, state):
        return state

    def __call__(self, *messages: Any) -> ReducerCall:
        if not messages:
            raise TypeError("a reducer binding requires at least one message")
        return ReducerCall(self, tuple(messages))

    def specialization_key(self) -> tuple[object, ...]:
        return (type(self).__qualname__, self.name, self.deterministic)


class SumReducer(Reducer):
    name = "sum"
    associative = True
    commutative = True

    def __init__(self, *, identity: float | int = 0, deterministic: bool = False) -> None:
        super().__init__(deterministic=deterministic)
        self.identity_value = identity

    def identity(self):
        return self.identity_value

    def combine(self, left, right):
        return left + right

    def specialization_key(self) -> tuple[object, ...]:
        return self.name, self.identity_value, self.deterministic


class OnlineSoftmaxReducer(Reducer):
    """Stable (maximum, denominator, numerator) softmax-weighted reducer."""

    name = "online_softmax"
    associative = True
    commutative = True

    def __init__(
        self,
        *,
        accumulation_dtype: object | None = None,
        deterministic: bool = False,
        block_prune_threshold: float | None = None,
    ) -> None:
        super().__init__(deterministic=deterministic)
        if block_prune_threshold is not None and not (
            0.0 < float(block_prune_threshold) <= 1.0
        ):
            raise ValueError("block_prune_threshold must be in (0, 1]")
        self.accumulation_dtype = accumulation_dtype
        self.block_prune_threshold = (
            None if block_prune_threshold is None else float(block_prune_threshold))

    def __call__(self, score: Any, value: Any) -> OnlineSoftmaxItem:
        return OnlineSoftmaxItem(score=score, value=value)

    def specialization_key(self) -> tuple[object, ...]:
        return (self.name, str(self.accumulation_dtype), self.deterministic,
                self.block_prune_threshold)


def sum(*, identity: float | int = 0, deterministic: bool = False) -> SumReducer:  # noqa: A001
    return SumReducer(identity=identity, deterministic=deterministic)


def online_softmax(
    *,
    accumulation_dtype: object | None = None,
    deterministic: bool = False,
    block_prune_threshold: float | None = None,
) -> OnlineSoftmaxReducer:
    return OnlineSoftmaxReducer(
        accumulation_dtype=accumulation_dtype,
        deterministic=deterministic,
        block_prune_threshold=block_prune_threshold,
    )


__all__ = [
    "OnlineSoftmaxItem",
    "OnlineSoftmaxReducer",
    "Reducer",
    "ReducerCall",
    "SumReducer",
    "online_softmax",
    "sum",
]

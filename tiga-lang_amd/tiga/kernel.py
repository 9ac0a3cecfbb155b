"""What a kernel ran, for ``explain()`` (reference python/tiga/kernel/model.py:99-229).

The public surface is the reference's observability API: ``last_variant``,
``variants``, ``explain()``, ``cache_info`` and ``CompiledVariant.code()``.
Here a variant is one (kernel, execution path, graph shape) combination: the
``hip`` backend with the libtgx_hip.so entry points it calls and the row
partition it uses, or ``torch-eager`` for an edge function no HIP kernel
covers.  ``cache_info`` counts calls: a *hit* is a warm call served by the
guarded launch of the previous call (no capture, recognition or
validation), a *miss* is a call that went through capture and dispatch.
"""

from __future__ import annotations

from dataclasses import dataclass, field


@dataclass(frozen=True)
class CompiledVariant:
    """One execution path a kernel took: backend, provider, the recognized
    edge-function pattern, how it is lowered, the entry points it calls and
    free-form remarks (row plan, reference planner decision)."""

    key: tuple[object, ...]
    backend: str
    provider: str
    pattern: str
    lowering: str | None = None
    entry_points: tuple[str, ...] = ()
    remarks: tuple[str, ...] = ()
    artifacts: dict[str, str] = field(default_factory=dict)

    def explain(self) -> str:
        calls = ", ".join(self.entry_points) or "(none)"
        text = [f"backend: {self.backend}", f"provider: {self.provider}",
                f"pattern: {self.pattern}", f"lowering: {self.lowering or '(unspecified)'}",
                f"entry points: {calls}"]
        text += [f"remark: {r}" for r in self.remarks]
        return "\n".join(text)

    def code(self, kind: str) -> str:
        """A stored artifact by kind.  The HIP provider is compiled ahead of
        time, so it keeps none and every kind raises KeyError."""
        if kind not in self.artifacts:
            raise KeyError(f"no {kind!r} artifact: provider {self.provider!r} keeps "
                           f"{sorted(self.artifacts) or 'none'}")
        return self.artifacts[kind]


class Kernel:
    """Base of ``MessagePassing``: the variants a kernel instance has run and
    its call counters."""

    def __init__(self) -> None:
        self._seen: dict[tuple[object, ...], CompiledVariant] = {}
        self._current: CompiledVariant | None = None
        self._warm_calls = 0
        self._cold_calls = 0

    @property
    def variants(self) -> tuple[CompiledVariant, ...]:
        return tuple(self._seen.values())

    @property
    def last_variant(self) -> CompiledVariant:
        if self._current is None:
            raise RuntimeError("kernel has not been called, so no variant exists")
        return self._current

    def explain(self) -> str:
        info = self.cache_info
        return (f"{self.last_variant.explain()}\n"
                f"variant cache: hits={info['hits']}, misses={info['misses']}")

    @property
    def cache_info(self) -> dict[str, int]:
        return {"hits": self._warm_calls, "misses": self._cold_calls,
                "variants": len(self._seen)}

    def _record_variant(self, variant: CompiledVariant) -> None:
        """A cold call ran `variant`."""
        self._cold_calls += 1
        self._seen[variant.key] = variant
        self._current = variant

    def _record_warm(self, variant: CompiledVariant) -> None:
        """A warm call re-ran `variant` through its guarded launch."""
        self._warm_calls += 1
        self._current = variant

"""Variant bookkeeping and ``explain()`` (reference python/tiga/kernel/model.py:99-229).

Each call records which execution path ran (``backend``: ``hip`` for the
gfx950 kernels, ``torch-eager`` for edge functions no HIP kernel covers), the
native entry points it used and the row-partition plan, so users can inspect
the chosen plan exactly as with the reference's ``kernel.explain()``.
"""

from __future__ import annotations

from dataclasses import dataclass, field


@dataclass(frozen=True)
class CompiledVariant:
    key: tuple[object, ...]
    backend: str
    provider: str
    pattern: str
    lowering: str | None = None
    entry_points: tuple[str, ...] = ()
    remarks: tuple[str, ...] = ()
    artifacts: dict[str, str] = field(default_factory=dict)

    def explain(self) -> str:
        lines = [
            f"backend: {self.backend}",
            f"provider: {self.provider}",
            f"pattern: {self.pattern}",
            f"lowering: {self.lowering or '(unspecified)'}",
            f"entry points: {', '.join(self.entry_points) if self.entry_points else '(none)'}",
        ]
        lines.extend(f"remark: {remark}" for remark in self.remarks)
        return "\n".join(lines)

    def code(self, kind: str) -> str:
        try:
            return self.artifacts[kind]
        except KeyError as exc:
            raise KeyError(
                f"artifact {kind!r} is unavailable for provider {self.provider!r}") from exc


class Kernel:
    def __init__(self) -> None:
        self._variants: dict[tuple[object, ...], CompiledVariant] = {}
        self._last_variant: CompiledVariant | None = None
        self._cache_hits = 0
        self._cache_misses = 0

    @property
    def variants(self) -> tuple[CompiledVariant, ...]:
        return tuple(self._variants.values())

    @property
    def last_variant(self) -> CompiledVariant:
        if self._last_variant is None:
            raise RuntimeError("kernel has not been called, so no variant exists")
        return self._last_variant

    def explain(self) -> str:
        return "\n".join((
            self.last_variant.explain(),
            f"variant cache: hits={self._cache_hits}, misses={self._cache_misses}",
        ))

    @property
    def cache_info(self) -> dict[str, int]:
        return {
            "hits": self._cache_hits,
            "misses": self._cache_misses,
            "variants": len(self._variants),
        }

    def _record_variant(self, variant: CompiledVariant) -> None:
        if variant.key in self._variants:
            self._cache_hits += 1
        else:
            self._cache_misses += 1
        self._variants[variant.key] = variant
        self._last_variant = variant

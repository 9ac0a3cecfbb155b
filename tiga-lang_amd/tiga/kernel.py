"""What a kernel ran, for ``explain()`` (reference python/tiga/kernel/model.py:99-229).

The public surface is the reference's observability API: ``last_variant``,
``variants``, ``explain()``, ``cache_info``, ``ir()``, ``code()``,
``diagnostics`` and ``schedules``.
Here a variant is one (kernel, execution path, graph shape) combination: the
``hip`` backend with the libtgx_hip.so entry points it calls and the row
partition it uses, or ``torch-eager`` for an edge function no HIP kernel
covers.  ``cache_info`` counts calls: a *hit* is a warm call served by the
guarded launch of the previous call (no capture, recognition or
validation), a *miss* is a call that went through capture and dispatch.
"""

from __future__ import annotations

from dataclasses import dataclass, field

_DISPOSITIONS = {"accepted", "rejected", "warning", "unknown", "remark"}


@dataclass(frozen=True)
class AnalysisFinding:
    """One structured diagnostic (the reference's finding record,
    kernel/model.py:8-27): here the planning remarks of a variant."""

    stage: str
    disposition: str
    message: str
    source_location: str | None = None
    affected_resource: str | None = None
    target_contract: str | None = None
    estimate: str | None = None
    suggested_action: str | None = None

    def __post_init__(self) -> None:
        if not self.stage or not self.message:
            raise ValueError("analysis findings require a stage and message")
        if self.disposition not in _DISPOSITIONS:
            raise ValueError("invalid analysis finding disposition")


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

    def ir(self, stage: str = "domain") -> str:
        """The variant's plan at `stage`.  This provider has no compiler IR:
        "domain" (or "domain-plan") is the recognized pattern, its lowering
        and entry points; other stages raise KeyError as in the reference."""
        if stage in ("domain", "domain-plan"):
            return self.explain()
        raise KeyError(f"IR/artifact stage {stage!r} is unavailable; have: domain")

    @property
    def diagnostics(self) -> tuple[AnalysisFinding, ...]:
        """The remarks as planning findings."""
        return tuple(AnalysisFinding("planning", "remark", r) for r in self.remarks)

    @property
    def schedules(self) -> tuple[object, ...]:
        """Verified machine schedules of the reference's compiler: none here
        (the HIP kernels are scheduled when the library is built)."""
        return ()


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

    def ir(self, stage: str = "domain") -> str:
        return self.last_variant.ir(stage)

    def code(self, kind: str = "ptx") -> str:
        return self.last_variant.code(kind)

    @property
    def diagnostics(self) -> tuple[AnalysisFinding, ...]:
        return self.last_variant.diagnostics

    @property
    def schedules(self) -> tuple[object, ...]:
        return self.last_variant.schedules

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

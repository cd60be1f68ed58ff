"""Per-sample accounting of the model-local PISA patches.

Interface of the reference's PISARuntimeState (pisa_runtime.py:12-153): the
same dataclass fields, record() / verify() / report() signatures and report
line (the runtime-report node and users parse it).  The state is a set of
counters behind one lock; record() maps each keyword it receives onto the
counter it feeds, verify() compares the per-layer hit counts with the counts
one forward per expected layer implies, and report() formats the counters.
Tensor data is never stored.
"""
from __future__ import annotations

from collections import Counter
from dataclasses import dataclass, field
from threading import Lock
from typing import Iterable

PISA_RUNTIME_ATTACHMENT = "rdna35_pisa_runtime_state"

_COUNTERS = ("per_layer_hits", "fallback_reasons", "shape_counts", "backend_counts", "hit_context_counts")


def _counts(counter: Counter) -> str:
    return ",".join(f"{key}:{value}" for key, value in sorted(counter.items())) or "-"


def _layer_range(start_layer: int, total_layers: int) -> tuple[int, ...]:
    if start_layer < 0 or total_layers < start_layer:
        raise ValueError("expected 0 <= start_layer <= total_layers")
    return tuple(range(start_layer, total_layers))


@dataclass
class PISARuntimeState:
    armed: bool = False
    executed: bool = False
    verified: bool = False
    failed: bool = False
    per_layer_hits: Counter = field(default_factory=Counter)
    fallback_reasons: Counter = field(default_factory=Counter)
    self_calls: int = 0
    cross_calls: int = 0
    shape_counts: Counter = field(default_factory=Counter)
    backend_counts: Counter = field(default_factory=Counter)
    hit_context_counts: Counter = field(default_factory=Counter)
    first_error: str | None = None
    quality_sample: str | None = None
    validated_profiles: set = field(default_factory=set)
    expected_layers: tuple = ()
    _expected: int | None = field(default=None, init=False, repr=False)
    _lock: Lock = field(default_factory=Lock, init=False, repr=False)

    @staticmethod
    def expected_calls(actual_forwards: int, start_layer: int = 20, total_layers: int = 28,
                       layers: Iterable[int] | None = None) -> int:
        """Patched-layer hits that `actual_forwards` forwards produce: one per layer per forward."""
        if actual_forwards < 0:
            raise ValueError("actual_forwards must be non-negative")
        chosen = _layer_range(start_layer, total_layers) if layers is None else tuple(layers)
        return actual_forwards * len(chosen)

    def reset(self, *, armed: bool | None = None) -> None:
        with self._lock:
            if armed is not None:
                self.armed = armed
            for name in _COUNTERS:
                getattr(self, name).clear()
            self.validated_profiles.clear()
            self.executed = self.verified = self.failed = False
            self.self_calls = self.cross_calls = 0
            self.first_error = self.quality_sample = None
            self._expected = None

    def _note_error(self, message: str) -> None:
        self.failed = True
        if self.first_error is None:
            self.first_error = message

    def record(self, *, layer: int | None = None, is_self_attention: bool | None = None,
               shape: Iterable[int] | None = None, fallback_reason: str | None = None,
               error: BaseException | str | None = None, backend: str | None = None, context: str | None = None,
               quality: str | None = None) -> None:
        """Account one attention dispatch from whichever of its facts the caller knows."""
        with self._lock:
            if is_self_attention is not None:
                if is_self_attention:
                    self.self_calls += 1
                else:
                    self.cross_calls += 1
            if shape is not None:
                self.shape_counts[tuple(map(int, shape))] += 1
            if fallback_reason is not None:
                self.fallback_reasons[str(fallback_reason)] += 1
            if error is not None:
                self._note_error(str(error))
            if backend is not None:
                self.backend_counts[str(backend)] += 1
                if context is not None:  # contexts are counted for hits, not for fallbacks
                    self.hit_context_counts[str(context)] += 1
            if quality is not None and self.quality_sample is None:
                self.quality_sample = str(quality)
            if layer is not None:
                self.per_layer_hits[int(layer)] += 1
                self.executed = True

    def verify(self, actual_forwards: int, start_layer: int = 20, total_layers: int = 28) -> bool:
        """True when every expected layer ran exactly `actual_forwards` times and nothing else ran or failed."""
        layers = tuple(self.expected_layers) or _layer_range(start_layer, total_layers)
        expected = self.expected_calls(actual_forwards, layers=layers)
        wanted = Counter({layer: actual_forwards for layer in layers})
        with self._lock:
            self._expected = expected
            hits = sum(self.per_layer_hits.values())
            observed = Counter({layer: n for layer, n in self.per_layer_hits.items() if n})
            ok = not self.failed and observed == +wanted
            if not ok and not self.failed:
                self._note_error(f"PISA hits={hits}, expected={expected}")
            self.verified = ok
            return ok

    def is_profile_validated(self, profile: tuple) -> bool:
        with self._lock:
            return profile in self.validated_profiles

    def mark_profile_validated(self, profile: tuple) -> None:
        with self._lock:
            self.validated_profiles.add(profile)

    def report(self) -> str:
        with self._lock:
            hits = sum(self.per_layer_hits.values())
            fields = (
                ("PISA armed", int(self.armed)), ("executed", int(self.executed)),
                ("verified", int(self.verified)), ("failed", int(self.failed)),
                ("hits", f"{hits}/{'?' if self._expected is None else self._expected}"),
                ("self", self.self_calls), ("cross", self.cross_calls),
                ("fallbacks", _counts(self.fallback_reasons)), ("backends", _counts(self.backend_counts)),
                ("hit_contexts", _counts(self.hit_context_counts)), ("shapes", _counts(self.shape_counts)),
                ("quality", self.quality_sample or "-"), ("first_error", self.first_error or "-"),
            )
        return " ".join(f"{name}={value}" for name, value in fields)

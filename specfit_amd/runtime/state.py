"""Cache key of one routed expert (src/specfit/state.py:7-15)."""
from __future__ import annotations

from dataclasses import dataclass, field


@dataclass(frozen=True, order=True, slots=True)
class ExpertKey:
    """(layer, expert) pair; ordered by layer first, then expert.  The hash
    is computed once (keys are looked up in the cache's maps on every
    expert access)."""

    layer_id: int
    expert_id: int
    _hash: int = field(init=False, repr=False, compare=False)

    def __post_init__(self) -> None:
        if self.layer_id < 0 or self.expert_id < 0:
            raise ValueError("layer_id and expert_id must be non-negative")
        object.__setattr__(self, "_hash", hash((self.layer_id, self.expert_id)))

    def __hash__(self) -> int:
        return self._hash

    def __eq__(self, other) -> bool:
        if other.__class__ is ExpertKey:
            return self.expert_id == other.expert_id and self.layer_id == other.layer_id
        return NotImplemented

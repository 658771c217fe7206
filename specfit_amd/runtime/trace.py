"""Cache transition kinds (src/specfit/trace.py:900-906)."""
from __future__ import annotations

from enum import Enum


class RuntimeEventKind(str, Enum):
    RESIDENT_HIT = "resident_hit"
    INFLIGHT_JOIN = "inflight_join"
    H2D_SUBMIT = "h2d_submit"
    EVICT = "evict"
    CONSUME_WAIT = "consume_wait"
    RELEASE = "release"

    def __str__(self) -> str:
        return self.value

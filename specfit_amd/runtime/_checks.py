"""Declarative field validation for the runtime's frozen records.

A record class lists its invariants as ``Rule`` rows (predicate over the
record, exception type, message); ``enforce`` raises the first rule that
fails, in table order.  The snapshot and cache-transition records use it,
so their invariants read as tables rather than as branches.
"""
from __future__ import annotations

from typing import Callable, NamedTuple


class Rule(NamedTuple):
    holds: Callable[[object], bool]
    error: type
    message: str


def count_rules(*names: str) -> tuple[Rule, ...]:
    """For each field: TypeError unless an int (bool excluded), then
    ValueError if negative -- field by field, in the order given."""
    rows = []
    for name in names:
        rows.append(Rule(lambda r, n=name: isinstance(getattr(r, n), int)
                         and not isinstance(getattr(r, n), bool),
                         TypeError, f"{name} must be an integer"))
        rows.append(Rule(lambda r, n=name: getattr(r, n) >= 0,
                         ValueError, f"{name} must be non-negative"))
    return tuple(rows)


def enforce(record, rules) -> None:
    for rule in rules:
        if not rule.holds(record):
            raise rule.error(rule.message)

"""Expert address (layer, expert); the record type of ``src/flash_moe/key.py:3-6``,
kept identical so reference callers can pass their keys unchanged."""
from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class ExpertKey:
    layer: int
    expert: int

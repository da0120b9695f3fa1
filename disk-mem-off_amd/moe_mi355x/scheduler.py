"""Prefetch schedulers (protocol of offload_runtime/scheduler/base.py:6-15).

``LookaheadScheduler`` keeps a fixed window: warm up the first ``lookahead`` layers and,
after layer ``i``, request layer ``i + lookahead`` (offload_runtime/scheduler/lookahead.py:6-23).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Protocol


class PrefetchScheduler(Protocol):
    def warmup_prefetch_ids(self, ordered_layer_ids: list[int]) -> list[int]: ...

    def next_prefetch_id(self, ordered_layer_ids: list[int], current_index: int) -> int | None: ...


@dataclass
class LookaheadScheduler:
    lookahead: int = 1

    def __post_init__(self) -> None:
        if self.lookahead < 0:
            raise ValueError("lookahead must be >= 0")

    def warmup_prefetch_ids(self, ordered_layer_ids: list[int]) -> list[int]:
        return list(ordered_layer_ids[: self.lookahead])

    def next_prefetch_id(self, ordered_layer_ids: list[int], current_index: int) -> int | None:
        if self.lookahead == 0:
            return None
        nxt = current_index + self.lookahead
        return ordered_layer_ids[nxt] if nxt < len(ordered_layer_ids) else None

"""Records exchanged with the KV allocator.

Same names, fields and validation as the reference boundary types
(reference src/pagedcore/engine_types.py:7-11 for the ids and tables,
:170-187 for KVReservation, :190-219 for CapacityCounts). The request-lifecycle
records of that module belong to the serving layer and are not part of this package.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import NewType, Tuple

RequestId = NewType("RequestId", str)
BlockId = NewType("BlockId", int)
BlockTable = Tuple[BlockId, ...]


@dataclass(frozen=True, slots=True)
class KVReservation:
    """Maximum block credits granted at admission, including blocks already owned.

    Credits do not assign physical blocks; blocks are taken from the pool only when
    tokens are appended (reference src/pagedcore/engine_types.py:170-187).
    """

    request_id: RequestId
    maximum_block_credits: int

    def __post_init__(self) -> None:
        credits = self.maximum_block_credits
        if not isinstance(credits, int) or isinstance(credits, bool) or credits <= 0:
            raise ValueError("maximum_block_credits must be a positive integer")


@dataclass(frozen=True, slots=True)
class CapacityCounts:
    """Pool occupancy snapshot (reference src/pagedcore/engine_types.py:190-219).

    Reserved credits overlap free capacity; owned blocks are also called occupied.
    """

    total_blocks: int
    free_blocks: int
    owned_blocks: int
    reserved_blocks: int
    active_slots: int
    live_cached_token_slots: int

    def __post_init__(self) -> None:
        for name in (
            "total_blocks",
            "free_blocks",
            "owned_blocks",
            "reserved_blocks",
            "active_slots",
            "live_cached_token_slots",
        ):
            value = getattr(self, name)
            if not isinstance(value, int) or isinstance(value, bool) or value < 0:
                raise ValueError(f"{name} must be a nonnegative integer")
        if self.free_blocks + self.owned_blocks != self.total_blocks:
            raise ValueError("free_blocks + owned_blocks must equal total_blocks")
        if not self.owned_blocks <= self.reserved_blocks <= self.total_blocks:
            raise ValueError("owned_blocks <= reserved_blocks <= total_blocks must hold")

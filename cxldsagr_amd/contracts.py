"""Attention selection and call contracts (the drop-in boundary for the DSA layer).

Mirrors ``models/attention_contracts.py:11-60`` and ``cache/contracts.py:11-31``
of the reference: the same dataclasses and Protocols, so an ``Indexer`` /
``MainAttention`` pair built here can stand in for the reference's.
"""

from dataclasses import dataclass
from typing import Any, Protocol

import torch


class CacheAccess(Protocol):
    """Committed token count and allocated token capacity for one request."""

    @property
    def length(self) -> int: ...

    @property
    def max_seq_len(self) -> int: ...

    def get_layer_state(self, layer_idx: int) -> object | None: ...

    def set_layer_state(self, layer_idx: int, state: object) -> None: ...


class CacheSession(Protocol):
    """Manager ownership independent of record storage and transfer backend."""

    @property
    def released(self) -> bool: ...

    def release(self) -> None: ...


@dataclass(frozen=True)
class BlockSelection:
    """Logical block IDs with shape [query, head_or_group, selected_block]."""

    block_ids: torch.Tensor
    block_size: int
    valid_mask: torch.Tensor | None = None


@dataclass(frozen=True)
class TokenSelection:
    """Logical token IDs with shape [query, selected_token]; -1 is padding.

    Token numbering is relative to the session. Constructing this value
    performs no tensor work.
    """

    token_ids: torch.Tensor


@dataclass(frozen=True)
class AttentionContext:
    layer_idx: int
    query_start: int
    query_length: int
    auxiliary_state: Any = None


class Indexer(Protocol):
    def __call__(
        self, q: torch.Tensor, cache_access: CacheAccess, context: AttentionContext
    ) -> BlockSelection | TokenSelection: ...


class MainAttention(Protocol):
    def __call__(
        self,
        q: torch.Tensor,
        selection: BlockSelection | TokenSelection | None,
        cache_access: CacheAccess,
        context: AttentionContext,
    ) -> torch.Tensor: ...

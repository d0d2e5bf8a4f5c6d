"""Pool-sizing configuration.

The subset of the reference's PagedCoreConfig (reference src/pagedcore/config.py:24-89)
that sizes the KV pool: the fields, their defaults, the integer/positivity checks and the
fixed 16-token block and 2048-token context are the same. Model identity, queue sizes,
networking and logging fields belong to the serving layer, which this package does not
include.
"""

from __future__ import annotations

from dataclasses import dataclass


class ConfigurationError(ValueError):
    pass


@dataclass(frozen=True, slots=True)
class PagedCoreConfig:
    context_limit: int = 2048
    block_tokens: int = 16
    kv_pool_mib: int = 8192
    workspace_margin_mib: int = 1536

    def __post_init__(self) -> None:
        for name in ("context_limit", "block_tokens", "kv_pool_mib", "workspace_margin_mib"):
            value = getattr(self, name)
            if not isinstance(value, int) or isinstance(value, bool):
                raise ConfigurationError(f"{name} must be an integer")
        if self.context_limit != 2048:
            raise ConfigurationError("context_limit is fixed at 2048")
        if self.block_tokens != 16:
            raise ConfigurationError("block_tokens is fixed at 16")
        for name in ("kv_pool_mib", "workspace_margin_mib"):
            if getattr(self, name) <= 0:
                raise ConfigurationError(f"{name} must be greater than zero")

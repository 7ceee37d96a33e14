from .orthogonalize import (
    OrthogonalizationStrategy,
    foreach_zeropower,
    foreach_zeropower_3d_fsdp,
    is_fsdp_3d_sharded,
    zeropower,
)

__all__ = [
    "OrthogonalizationStrategy",
    "foreach_zeropower",
    "foreach_zeropower_3d_fsdp",
    "is_fsdp_3d_sharded",
    "zeropower",
]

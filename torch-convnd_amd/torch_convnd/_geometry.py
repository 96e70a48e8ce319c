"""Spatial argument helpers shared by the functional and module frontends."""

from collections.abc import Sequence

# The reference's default patch-buffer cap (src/torch_convnd/_geometry.py:5). The gfx950
# kernels need no patch buffer but keep validating the contract.
DEFAULT_WORKSPACE_BYTES = 64 * 1024 * 1024


def any_true(values: list) -> bool:
    """``any`` over a list, written as a loop so every Dynamo release traces it."""
    for value in values:
        if value:
            return True
    return False


def has_rank(ndim: int, rank: int) -> bool:
    """Whether ``ndim`` dimensions hold a batched or an unbatched rank-``rank`` input."""
    return ndim == rank + 2 or ndim == rank + 1


def _tuple(value: int | Sequence[int], rank: int, name: str) -> tuple[int, ...]:
    """Broadcast an int to ``rank`` entries or check a sequence of exactly ``rank`` ints."""
    if isinstance(value, int) and not isinstance(value, bool):
        return (value,) * rank
    if isinstance(value, (str, bytes)) or not isinstance(value, Sequence):
        raise TypeError(f"{name} must be an integer or a sequence of integers")
    items = tuple(value)
    bad = [not isinstance(item, int) or isinstance(item, bool) for item in items]
    if len(items) != rank or any_true(bad):
        raise ValueError(f"{name} must contain exactly {rank} integers")
    return items

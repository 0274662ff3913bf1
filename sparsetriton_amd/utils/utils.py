"""Argument helpers."""

from typing import Any, List, Tuple, Union

__all__ = ["make_ntuple"]


def make_ntuple(value: Union[int, float, Tuple[Any, ...], List[Any]], n: int) -> Tuple[Any, ...]:
    """Expand a scalar to an n-tuple; truncate or right-pad (with the last item) a sequence.

    Same behaviour as ``sparsetriton/utils/utils.py:17-47``.
    """
    if isinstance(value, (list, tuple)):
        if len(value) >= n:
            return tuple(value[:n])
        return tuple(value) + (value[-1],) * (n - len(value))
    if isinstance(value, (int, float)):
        return (value,) * n
    raise TypeError(f"Expected int, float, tuple, or list, got {type(value)}")

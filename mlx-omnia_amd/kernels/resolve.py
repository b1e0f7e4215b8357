"""The one resolution rule every primitive's facade shares (core/kernels/resolve.py:32-38).

A primitive's `_STRATEGIES` is an ordered tuple of strategy classes; `resolve` hands each
`build` the full declaration and the first one that returns an instance wins. The last
entry of every tuple is a Core strategy that accepts every declaration, so resolution is
total. `RESOLVED` records the modules of the strategies that actually built in this
process (core/kernels/resolve.py:25-29), which is how a test or a bench line proves
which binding executed.
"""

from __future__ import annotations

from collections.abc import Iterable
from typing import Any, Protocol, TypeVar

S = TypeVar("S", covariant=True)


class Builds(Protocol[S]):
    def build(self, *args: Any, **kwargs: Any) -> S | None: ...


RESOLVED: set[str] = set()


def resolve(strategies: Iterable[Builds[S]], /, *args: Any, **kwargs: Any) -> S:
    """Order is preference: the first strategy that builds wins."""
    built = next(
        built for strategy in strategies if (built := strategy.build(*args, **kwargs)) is not None
    )
    RESOLVED.add(type(built).__module__)
    return built

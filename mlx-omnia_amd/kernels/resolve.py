"""The one resolution rule every primitive's facade shares (core/kernels/resolve.py:32-38).

A primitive's `_STRATEGIES` is an ordered tuple of strategy classes; `resolve` hands each
`build` the full declaration and the first one that returns an instance wins. The last
entry of every tuple is a Core strategy that accepts every declaration, so resolution is
total. `RESOLVED` records the modules of the strategies that actually built in this
process (core/kernels/resolve.py:25-29), which is how a test or a bench line proves
which binding executed. A HIP strategy that hands one call to its Core chain (an input
its kernel does not take, seen only at call time) records it with `record_fallback`:
the Core module joins `RESOLVED` and the hand-off is counted in `FALLBACKS`.
"""

from __future__ import annotations

from collections.abc import Iterable
from typing import Any, Protocol, TypeVar

S = TypeVar("S", covariant=True)


class Builds(Protocol[S]):
    def build(self, *args: Any, **kwargs: Any) -> S | None: ...


RESOLVED: set[str] = set()
FALLBACKS: dict[str, int] = {}


def resolve(strategies: Iterable[Builds[S]], /, *args: Any, **kwargs: Any) -> S:
    """The instance from the earliest strategy in `strategies` whose `build` accepts."""
    built = next(
        built for strategy in strategies if (built := strategy.build(*args, **kwargs)) is not None
    )
    RESOLVED.add(type(built).__module__)
    return built


def record_fallback(strategy: object, core: object) -> None:
    """Note that `strategy` (a built HIP binding) passed a call to its Core chain `core`."""
    RESOLVED.add(type(core).__module__)
    name = f"{type(strategy).__name__} -> {type(core).__name__}"
    FALLBACKS[name] = FALLBACKS.get(name, 0) + 1

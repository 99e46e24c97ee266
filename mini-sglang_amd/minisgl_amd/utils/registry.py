"""Name -> creator registry (same contract as python/minisgl/utils/registry.py:6-38)."""

from __future__ import annotations

from typing import Callable, Dict, Generic, Iterable, List, TypeVar

T = TypeVar("T")


class Registry(Generic[T]):
    def __init__(self, kind: str):
        self._items: Dict[str, T] = {}
        self._kind = kind

    def register(self, name: str) -> Callable[[T], T]:
        if name in self._items:
            raise KeyError(f"{self._kind} '{name}' is already registered.")

        def decorator(item: T) -> T:
            self._items[name] = item
            return item

        return decorator

    def __getitem__(self, name: str) -> T:
        if name not in self._items:
            raise KeyError(f"Unsupported {self._kind}: {name}")
        return self._items[name]

    def supported_names(self) -> List[str]:
        return list(self._items)

    def assert_supported(self, names: str | Iterable[str]) -> None:
        if isinstance(names, str):
            names = [names]
        for name in names:
            if name not in self._items:
                from argparse import ArgumentTypeError

                raise ArgumentTypeError(
                    f"Unsupported {self._kind}: {name}. Supported items: {self.supported_names()}"
                )

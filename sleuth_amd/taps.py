"""Named observation points ("taps") of the attention module.

The module exposes four of them (names relative to the module; the reference's tap
contract, sleuth/forge/model/taps.py:22-34):
    q        queries after norm + RoPE          [B, H, T, hd]
    k        keys after norm + RoPE (KV heads)  [B, K, T, hd]
    pattern  attention probabilities           [B, H, T, S]  (listening forces the torch path)
    z        per-head attention output         [B, T, H, hd]
A listener is called as fn(name, tensor); a tensor it returns replaces the activation.

Interoperability: when the module runs inside Sleuth (the package `sleuth.forge.model.taps`
is importable), `tap_class()` is the host's own Tap type, so the host's isinstance-based
discovery (taps.py:68-102: assign_tap_names / listen) sees the attention taps like any
other. Outside Sleuth the module uses `Tap` below. The helpers in this file (name_taps,
listen, tap_names) find taps by duck typing -- any module with `name` and a `listeners`
list -- so they work on either kind.
"""

from __future__ import annotations

import fnmatch
import functools
import importlib
from contextlib import ExitStack, contextmanager
from typing import Callable, Iterator

import torch
from torch import nn

Listener = Callable[[str, torch.Tensor], "torch.Tensor | None"]
HOST_TAPS_MODULE = "sleuth.forge.model.taps"


class Tap(nn.Module):
    """Identity module with a name; `listeners` is a plain list so that a host analyzer
    that appends to it (the reference's protocol) and `listen()` below both work."""

    def __init__(self) -> None:
        super().__init__()
        self.name = "<unnamed>"
        self.listeners: list[Listener] = []

    @property
    def active(self) -> bool:
        return len(self.listeners) > 0

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if not self.listeners:
            return x
        for fn in tuple(self.listeners):   # a listener may detach itself
            replaced = fn(self.name, x)
            x = x if replaced is None else replaced
        return x

    def extra_repr(self) -> str:
        return repr(self.name)


@functools.lru_cache(maxsize=None)
def tap_class() -> type:
    """The Tap type new modules are built with: the host's when Sleuth is importable,
    else this file's. Cached; tests that swap the host call tap_class.cache_clear()."""
    try:
        host = importlib.import_module(HOST_TAPS_MODULE)
    except ImportError:
        return Tap
    cls = getattr(host, "Tap", None)
    return cls if isinstance(cls, type) and issubclass(cls, nn.Module) else Tap


def make_tap() -> nn.Module:
    return tap_class()()


def is_tap(m: nn.Module) -> bool:
    return isinstance(getattr(m, "listeners", None), list) and hasattr(m, "name")


def tap_active(t: nn.Module) -> bool:
    """Whether anything listens on t (either kind of tap)."""
    return bool(getattr(t, "listeners", None))


def _iter_taps(model: nn.Module) -> Iterator[tuple[str, nn.Module]]:
    for path, m in model.named_modules():
        if is_tap(m):
            yield path, m


def name_taps(model: nn.Module) -> None:
    """Name every tap after its place in the tree, the attribute's `tap_` prefix dropped:
    blocks.3.attn.tap_z is named blocks.3.attn.z (the reference's naming rule)."""
    for path, t in _iter_taps(model):
        head, _, leaf = path.rpartition(".")
        if leaf.startswith("tap_"):
            leaf = leaf[len("tap_"):]
        t.name = f"{head}.{leaf}" if head else leaf


assign_tap_names = name_taps   # the reference's name for the same operation


def tap_names(model: nn.Module) -> list[str]:
    return [t.name for _, t in _iter_taps(model)]


def find_taps(model: nn.Module, pattern: str) -> list[nn.Module]:
    hits = [t for _, t in _iter_taps(model) if fnmatch.fnmatchcase(t.name, pattern)]
    if not hits:
        raise KeyError(f"no tap matches {pattern!r}")
    return hits


@contextmanager
def listen(model: nn.Module, listeners: dict[str, Listener]) -> Iterator[None]:
    """Attach fn to every tap whose name matches its pattern for the `with` block; every
    attachment is undone on exit, also when the block raises."""
    with ExitStack() as undo:
        for pattern, fn in listeners.items():
            for t in find_taps(model, pattern):
                t.listeners.append(fn)
                undo.callback(t.listeners.remove, fn)
        yield

"""Taps: named identity points the analyzer can listen on or replace.

Same contract as sleuth/forge/model/taps.py:47-102: a Tap calls each listener as
fn(name, tensor) and a returned tensor replaces the activation; listen() attaches
listeners by fnmatch pattern for the duration of a `with` block. The attention module
exposes attn.q / attn.k ([B,H,T,hd] after RoPE), attn.pattern ([B,H,T,S] probabilities;
listening forces the explicit torch path) and attn.z ([B,T,H,hd] per-head output).
"""

from __future__ import annotations

import fnmatch
from contextlib import contextmanager
from typing import Callable, Iterator

import torch
from torch import nn

Listener = Callable[[str, torch.Tensor], "torch.Tensor | None"]


class Tap(nn.Module):
    def __init__(self):
        super().__init__()
        self.name = "<unnamed>"
        self.listeners: list[Listener] = []

    @property
    def active(self) -> bool:
        return bool(self.listeners)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        for fn in self.listeners:
            out = fn(self.name, x)
            if out is not None:
                x = out
        return x


def assign_tap_names(model: nn.Module) -> None:
    """blocks.3.attn.tap_z -> blocks.3.attn.z"""
    for path, m in model.named_modules():
        if isinstance(m, Tap):
            parts = path.split(".")
            parts[-1] = parts[-1].removeprefix("tap_")
            m.name = ".".join(parts)


def find_taps(model: nn.Module, pattern: str) -> list[Tap]:
    taps = [m for m in model.modules() if isinstance(m, Tap) and fnmatch.fnmatchcase(m.name, pattern)]
    if not taps:
        raise KeyError(f"no tap matches {pattern!r}")
    return taps


def tap_names(model: nn.Module) -> list[str]:
    return [m.name for m in model.modules() if isinstance(m, Tap)]


@contextmanager
def listen(model: nn.Module, listeners: dict[str, Listener]) -> Iterator[None]:
    attached: list[tuple[Tap, Listener]] = []
    try:
        for pattern, fn in listeners.items():
            for tap in find_taps(model, pattern):
                tap.listeners.append(fn)
                attached.append((tap, fn))
        yield
    finally:
        for tap, fn in attached:
            tap.listeners.remove(fn)

"""ActivationQuantMode / ActivationQuantConfig, as in the reference's
src/activation_quant.rs:7-44 (default mode Off; `strict` rejects paths that are
not implemented; is_enabled() is true for any mode but Off)."""

from __future__ import annotations

import enum
from dataclasses import dataclass, field


class ActivationQuantMode(enum.IntEnum):
    Off = 0   # floating-point activations
    W8A8 = 1  # per-row int8 fake quantisation of x
    W4A8 = 2  # contract only; runs as Off unless strict

    @classmethod
    def default(cls) -> "ActivationQuantMode":
        return cls.Off


@dataclass(frozen=True)
class ActivationQuantConfig:
    mode: ActivationQuantMode = field(default=ActivationQuantMode.Off)
    strict: bool = False

    def is_enabled(self) -> bool:
        return self.mode != ActivationQuantMode.Off

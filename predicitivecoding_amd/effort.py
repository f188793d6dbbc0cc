"""Named inference-effort tiers, the host mirror of
PredicitiveCoding/Networks/EffortLevel.cs: each level pairs a step budget with
the relative early-exit threshold of adaptive settling (EffortPresets.For,
EffortLevel.cs:33-39), as PcDeviceModel.predict_adaptive takes them.
"""
from __future__ import annotations

from enum import Enum

from .errors import ArgumentOutOfRangeException


class EffortLevel(Enum):
    """EffortLevel.cs:14-22."""
    Low = 0
    Medium = 1
    High = 2


class EffortPresets:
    _TABLE = {EffortLevel.Low: (10, 1e-3), EffortLevel.Medium: (30, 1e-4), EffortLevel.High: (100, 1e-5)}

    @staticmethod
    def for_level(level: EffortLevel) -> tuple[int, float]:
        """(max_steps, epsilon) of a level; an unknown level raises as the
        reference's switch does (EffortLevel.cs:38)."""
        if level not in EffortPresets._TABLE:
            raise ArgumentOutOfRangeException("level")
        return EffortPresets._TABLE[level]

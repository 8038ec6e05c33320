"""Controller button masks and the discrete action sets of the trainers.

A mask has one bit per NES pad button, in the order the pad shifts them out
(A first): A=0, B=1, SELECT=2, START=3, UP=4, DOWN=5, LEFT=6, RIGHT=7 -- the
reference's ``Button`` enum and ``encode_action`` (src/nesle/actions.py:7-45).
The action sets are the reference's (actions.py:48-104); ``COMPLEX_MOVEMENT``
is the 12-way space of the PPO workload.
"""

from __future__ import annotations

from enum import IntEnum
from typing import Iterable


class Button(IntEnum):
    A = 0
    B = 1
    SELECT = 2
    START = 3
    UP = 4
    DOWN = 5
    LEFT = 6
    RIGHT = 7


_NAMES = {b.name.lower(): b for b in Button}
_NOOP = {"noop", "no-op", "none"}


def encode_action(buttons: Iterable[str | Button]) -> int:
    """Button names (case-insensitive; "NOOP" adds nothing) or Buttons -> mask."""
    mask = 0
    for button in buttons:
        if isinstance(button, Button):
            mask |= 1 << int(button)
            continue
        key = str(button).strip().lower()
        if key in _NOOP:
            continue
        if key not in _NAMES:
            raise ValueError(f"unknown NES controller button: {button!r}")
        mask |= 1 << int(_NAMES[key])
    return mask


RIGHT_ONLY = [["NOOP"], ["right"], ["right", "A"], ["right", "B"], ["right", "A", "B"]]
SIMPLE_MOVEMENT = RIGHT_ONLY + [["A"], ["left"]]
SIMPLE_MOVEMENT_WITH_START = [["start"], *SIMPLE_MOVEMENT]
COMPLEX_MOVEMENT = SIMPLE_MOVEMENT + [["left", "A"], ["left", "B"], ["left", "A", "B"], ["down"], ["up"]]
MARIO_MOVEMENT = [["NOOP"], ["right"], ["right", "B"], ["right", "A"], ["right", "B", "A"], ["A"], ["B", "A"],
                  ["left"], ["left", "A"], ["down"], ["right", "down"]]

RIGHT_ONLY_MASKS = tuple(encode_action(a) for a in RIGHT_ONLY)
SIMPLE_MOVEMENT_MASKS = tuple(encode_action(a) for a in SIMPLE_MOVEMENT)
SIMPLE_MOVEMENT_WITH_START_MASKS = tuple(encode_action(a) for a in SIMPLE_MOVEMENT_WITH_START)
COMPLEX_MOVEMENT_MASKS = tuple(encode_action(a) for a in COMPLEX_MOVEMENT)
MARIO_MOVEMENT_MASKS = tuple(encode_action(a) for a in MARIO_MOVEMENT)


def action_masks(action_space) -> tuple[int, ...]:
    """Action-space name or explicit masks -> masks (src/nesle/env.py:119-138)."""
    if isinstance(action_space, str):
        key = action_space.lower().replace("-", "_")
        if key in {"right", "right_only"}:
            return RIGHT_ONLY_MASKS
        if key == "simple":
            return SIMPLE_MOVEMENT_MASKS
        if key in {"simple_with_start", "simple_start"}:
            return SIMPLE_MOVEMENT_WITH_START_MASKS
        if key == "complex":
            return COMPLEX_MOVEMENT_MASKS
        if key == "mario":
            return MARIO_MOVEMENT_MASKS
        if key in {"full", "raw"}:
            return tuple(range(256))
        raise ValueError(f"unknown action space: {action_space!r}")
    masks = tuple(int(m) & 0xFF for m in action_space)
    if not masks:
        raise ValueError("custom action space must contain at least one action mask")
    return masks

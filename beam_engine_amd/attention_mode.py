"""Prefill / decode switch of the model forward (src/beam_engine/attention_mode.py:7-15)."""

from enum import Enum


class AttentionMode(Enum):
    PREFILL = "prefill"
    DECODE = "decode"

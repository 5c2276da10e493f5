"""Seeded per-head pattern configs in the reference's JSON format.

Format (parsed as-is by minference_forward.load_layer_patterns, reference
minference/modules/minference_forward.py:187-198): a list with one dict per
layer mapping ``str(head)`` to ``[type, p1, p2, score]``:
  ["stream_llm", n_init, n_local, score] | ["block_sparse", topk, 0, score] |
  ["dense", 0, 0, score]

``mixed_config`` draws a fixed-count mix over all layer*head slots from a
seed, which is how the synthetic Phi-3 benchmark mixes are defined
(e.g. 30% stream / 60% block / 10% dense).
"""

from __future__ import annotations

import json
import random
from typing import List, Sequence, Tuple

NUM_LAYERS_PHI3 = 32
NUM_HEADS_PHI3 = 32


def record(kind: str, p1: int = 0, p2: int = 0, score: float = 1.0) -> list:
    if kind not in ("stream_llm", "block_sparse", "dense"):
        raise ValueError(f"unknown pattern kind {kind!r}")
    return [kind, int(p1), int(p2), float(score)]


def uniform_config(kind: str, p1: int = 0, p2: int = 0, n_layers: int = NUM_LAYERS_PHI3,
                   n_heads: int = NUM_HEADS_PHI3) -> List[dict]:
    return [{str(h): record(kind, p1, p2) for h in range(n_heads)} for _ in range(n_layers)]


def mixed_config(mix: Sequence[Tuple[float, list]], seed: int = 0,
                 n_layers: int = NUM_LAYERS_PHI3, n_heads: int = NUM_HEADS_PHI3) -> List[dict]:
    """``mix`` = [(fraction, record), ...]; counts are round(fraction * total)
    with the remainder going to the last entry, assigned by a seeded shuffle."""
    total = n_layers * n_heads
    counts = [int(round(f * total)) for f, _ in mix]
    counts[-1] = total - sum(counts[:-1])
    if min(counts) < 0:
        raise ValueError("mix fractions exceed 1")
    slots = []
    for c, (_, rec) in zip(counts, mix):
        slots += [rec] * c
    random.Random(seed).shuffle(slots)
    out = []
    for layer in range(n_layers):
        out.append({str(h): list(slots[layer * n_heads + h]) for h in range(n_heads)})
    return out


def headline_config(seed: int = 0, n_layers: int = NUM_LAYERS_PHI3,
                    n_heads: int = NUM_HEADS_PHI3) -> List[dict]:
    """All heads sparse: 50% stream_llm(128, 4096), 50% block_sparse(top-100)."""
    return mixed_config([(0.5, record("stream_llm", 128, 4096)),
                         (0.5, record("block_sparse", 100, 0))], seed, n_layers, n_heads)


def write(path: str, cfg: List[dict]) -> None:
    with open(path, "w") as f:
        json.dump(cfg, f, indent=1)
        f.write("\n")

"""Seeded per-head pattern configs in the reference's JSON format.

Format (parsed as-is by minference_forward.load_layer_patterns, reference
minference/modules/minference_forward.py:187-198): a list with one dict per
layer mapping ``str(head)`` to ``[type, p1, p2, score]``:
  ["stream_llm", n_init, n_local, score] | ["block_sparse", topk, 0, score] |
  ["dense", 0, 0, score] | ["vertical_and_slash", n_vertical, n_slash, score]
A head missing from its layer dict, and every head of a missing layer, runs
the default record ("vertical_and_slash", 1000, 6096, 1) (reference :404-407).

``mixed_config`` draws a fixed-count mix over all layer*head slots from a
seed, which is how the synthetic Phi-3 benchmark mixes are defined
(e.g. 30% stream / 60% block / 10% dense).  ``probe_config``,
``layer_range_config`` and the range parsers build the probe and sweep files
of reference benchmarks/prepare_phi3_pathb_configs.py:96-193;
``validate_config`` checks a file against the format and the dispatcher's
rules before a model loads it.
"""

from __future__ import annotations

import collections
import json
import numbers
import random
from dataclasses import dataclass, field
from typing import Dict, Iterable, List, Optional, Sequence, Tuple

NUM_LAYERS_PHI3 = 32
NUM_HEADS_PHI3 = 32

KINDS = ("stream_llm", "block_sparse", "dense", "vertical_and_slash")

# Record a head gets when the file does not name it (reference
# minference_forward.py:404-407).
DEFAULT_RECORD = ("vertical_and_slash", 1000, 6096, 1)


def record(kind: str, p1: int = 0, p2: int = 0, score: float = 1.0) -> list:
    if kind not in KINDS:
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


def write(path: str, cfg: List[dict], indent: int = 1) -> None:
    with open(path, "w") as f:
        json.dump(cfg, f, indent=indent)
        f.write("\n")


def load(path: str, n_layers: Optional[int] = NUM_LAYERS_PHI3,
         n_heads: Optional[int] = NUM_HEADS_PHI3) -> List[dict]:
    """Read a pattern file and validate it (raises PatternConfigError)."""
    with open(path) as f:
        cfg = json.load(f)
    validate_config(cfg, n_layers, n_heads, where=path)
    return cfg


# ---------------------------------------------------------------------------
# probe and sweep files (reference benchmarks/prepare_phi3_pathb_configs.py)
# ---------------------------------------------------------------------------
def heads_of(cfg: Sequence[dict], kind: str) -> List[Tuple[int, int, float]]:
    """(layer, head, score) of every head whose record has type ``kind``,
    layer-major and head-ascending.  Applied to the original Phi-3 best
    pattern with kind "stream_llm" this yields the 43 probe target heads of
    the reference's probe files (prepare_phi3_pathb_configs.py:49-93)."""
    out = []
    for layer, heads in enumerate(cfg):
        for h in sorted(heads, key=int):
            rec = heads[h]
            if rec[0] == kind:
                out.append((layer, int(h), rec[3]))
    return out


def probe_config(targets: Iterable[Sequence], rec: Sequence, others: Sequence = None,
                 n_layers: int = NUM_LAYERS_PHI3, n_heads: int = NUM_HEADS_PHI3) -> List[dict]:
    """Every head runs ``others`` (default dense) except the ``targets``
    ((layer, head) or (layer, head, score)), which run ``rec`` with the
    target's score when one is given (reference :96-116)."""
    base = list(record("dense") if others is None else others)
    out = [{str(h): list(base) for h in range(n_heads)} for _ in range(n_layers)]
    for t in targets:
        layer, head = int(t[0]), int(t[1])
        if not (0 <= layer < n_layers and 0 <= head < n_heads):
            raise ValueError(f"probe target (layer={layer}, head={head}) outside "
                             f"{n_layers} layers x {n_heads} heads")
        r = list(rec)
        if len(t) > 2:
            r[3] = t[2]
        out[layer][str(head)] = r
    return out


def layer_range_config(layers: Iterable[int], rec: Sequence, others: Sequence = None,
                       n_layers: int = NUM_LAYERS_PHI3,
                       n_heads: int = NUM_HEADS_PHI3) -> List[dict]:
    """All heads of ``layers`` run ``rec``, every other layer ``others``
    (default dense) (reference :119-136)."""
    chosen = set(int(x) for x in layers)
    bad = [x for x in chosen if not 0 <= x < n_layers]
    if bad:
        raise ValueError(f"layers {sorted(bad)} outside [0, {n_layers})")
    base = list(record("dense") if others is None else others)
    return [{str(h): list(rec if layer in chosen else base) for h in range(n_heads)}
            for layer in range(n_layers)]


def parse_layer_range(spec: str, n_layers: int = NUM_LAYERS_PHI3) -> Tuple[int, int]:
    """``"8-13"`` -> (8, 13) inclusive, ``"8"`` -> (8, 8); ValueError when the
    range is empty or leaves [0, n_layers) (reference :146-158)."""
    text = spec.strip()
    lo_s, sep, hi_s = text.partition("-")
    try:
        lo = int(lo_s)
        hi = int(hi_s) if sep else lo
    except ValueError:
        raise ValueError(f"layer range {spec!r} is not 'lo-hi' or 'layer'") from None
    if not 0 <= lo <= hi < n_layers:
        raise ValueError(f"layer range {spec!r} out of [0, {n_layers - 1}] or lo > hi")
    return lo, hi


def parse_layer_ranges(csv: str, n_layers: int = NUM_LAYERS_PHI3) -> List[Tuple[int, int]]:
    return [parse_layer_range(x, n_layers) for x in csv.split(",") if x.strip()]


def parse_topks(csv: str) -> List[int]:
    """Comma-separated top-k values, each >= 1 (reference :167-180)."""
    out = []
    for x in csv.split(","):
        if x.strip():
            v = int(x)
            if v < 1:
                raise ValueError(f"topk must be >= 1, got {v}")
            out.append(v)
    return out


PATHB_PREFIX = "Phi_3_mini_128k_instruct_pathb_"


def layer_range_name(lo: int, hi: int, topk: int) -> str:
    """File name the reference gives a layer-range block_sparse sweep file
    (:183-187), so scripts that pass those paths find them."""
    return f"{PATHB_PREFIX}block_sparse_layers{lo}_{hi}_all_heads_topk{topk}_latency.json"


def pathb_configs(targets: Sequence[Sequence], n_init: int = 128, n_local: int = 896,
                  topk_blocks: int = 16, probe_topks: Sequence[int] = (1, 2, 4),
                  layer_ranges: Sequence[Tuple[int, int]] = ((8, 13),),
                  range_topks: Sequence[int] = (1, 2, 4)) -> Dict[str, List[dict]]:
    """The reference's default probe and sweep file set keyed by file name
    (prepare_phi3_pathb_configs.py:213-300 with its default arguments):
    stream_llm(n_init, n_local) and block_sparse(topk_blocks) on the probe
    targets with the other heads dense, block_sparse probes at each of
    ``probe_topks``, every head block_sparse(topk_blocks), and each layer
    range at each of ``range_topks``."""
    if n_init % 64 or n_local % 64:
        raise ValueError("n_init and n_local must be multiples of 64")
    if topk_blocks < 1 or min(list(probe_topks) + list(range_topks) + [1]) < 1:
        raise ValueError("top-k values must be >= 1")
    out = {
        PATHB_PREFIX + "stream_llm_aligned_dense_others.json":
            probe_config(targets, record("stream_llm", n_init, n_local)),
        PATHB_PREFIX + "block_sparse_probe_dense_others.json":
            probe_config(targets, record("block_sparse", topk_blocks)),
        PATHB_PREFIX + "block_sparse_all_heads_latency.json":
            uniform_config("block_sparse", topk_blocks),
    }
    for t in probe_topks:
        out[PATHB_PREFIX + f"block_sparse_probe_dense_others_topk{t}.json"] = \
            probe_config(targets, record("block_sparse", t))
    for lo, hi in layer_ranges:
        for t in range_topks:
            out[layer_range_name(lo, hi, t)] = \
                layer_range_config(range(lo, hi + 1), record("block_sparse", t))
    return out


# ---------------------------------------------------------------------------
# validation
# ---------------------------------------------------------------------------
class PatternConfigError(ValueError):
    """A pattern file that the dispatcher would reject or misread."""


@dataclass
class ConfigSummary:
    """What a validated file asks for over ``n_layers`` x ``n_heads`` heads.

    counts[(type, p1, p2)] = heads, defaulted heads included; ``defaulted`` =
    heads the file does not name; ``notes`` = legal records whose parameters
    the dispatcher clamps or that leave rows with nothing to attend."""

    n_layers: int
    n_heads: int
    counts: Dict[Tuple[str, int, int], int] = field(default_factory=dict)
    defaulted: int = 0
    notes: List[str] = field(default_factory=list)

    def kind_counts(self) -> Dict[str, int]:
        c: Dict[str, int] = collections.Counter()
        for (kind, _, _), n in self.counts.items():
            c[kind] += n
        return dict(c)


def _as_int(x) -> Optional[int]:
    """int(x) for ints and integral floats (the dispatcher calls int() on the
    parameters, :409-414); None for anything else, bools included."""
    if isinstance(x, bool):
        return None
    if isinstance(x, numbers.Integral):
        return int(x)
    if isinstance(x, float) and x.is_integer():
        return int(x)
    return None


def validate_config(cfg, n_layers: Optional[int] = NUM_LAYERS_PHI3,
                    n_heads: Optional[int] = NUM_HEADS_PHI3, *,
                    where: str = "pattern config") -> ConfigSummary:
    """Check a parsed pattern file; raise PatternConfigError listing every
    problem, each with its layer and head.

    Errors are what the dispatcher (reference minference_forward.py:187-198,
    :404-419) would fail on or silently misread: a file that is not a list of
    dicts, head keys that are not decimal head numbers in [0, n_heads),
    records that are not 4-element lists, unknown types, non-integer
    parameters, a non-numeric score, negative stream_llm windows, and more
    layers than the model has.  Legal values the dispatcher clamps
    (block_sparse top-k < 1, vertical_and_slash sizes below 30/50) and
    stream_llm(n_init, 0) heads, whose rows past n_init see no key, are
    reported in ``notes``.  ``n_layers`` / ``n_heads`` = None skip the
    corresponding range checks."""
    errors: List[str] = []
    if not isinstance(cfg, list):
        raise PatternConfigError(f"{where}: top level must be a list of per-layer dicts, "
                                 f"got {type(cfg).__name__}")
    if n_layers is not None and len(cfg) > n_layers:
        errors.append(f"{len(cfg)} layers, the model has {n_layers}")
    heads_total = n_heads if n_heads is not None else 0
    summary = ConfigSummary(len(cfg) if n_layers is None else n_layers, heads_total)
    counts: Dict[Tuple[str, int, int], int] = collections.Counter()
    for layer, heads in enumerate(cfg):
        if not isinstance(heads, dict):
            errors.append(f"layer {layer}: expected a dict of head records, "
                          f"got {type(heads).__name__}")
            continue
        named = set()
        for key, rec in heads.items():
            at = f"layer {layer} head {key!r}"
            if not (isinstance(key, str) and key.isascii() and key.isdigit()):
                errors.append(f"{at}: head key must be a decimal head number")
                continue
            h = int(key)
            if n_heads is not None and h >= n_heads:
                errors.append(f"{at}: head {h} >= {n_heads} heads")
                continue
            if h in named:
                errors.append(f"{at}: head {h} named twice")
                continue
            named.add(h)
            if not isinstance(rec, (list, tuple)) or len(rec) != 4:
                errors.append(f"{at}: record must be [type, p1, p2, score], got {rec!r}")
                continue
            kind, p1, p2, score = rec
            if kind not in KINDS:
                errors.append(f"{at}: unknown pattern type {kind!r} (one of {', '.join(KINDS)})")
                continue
            i1, i2 = _as_int(p1), _as_int(p2)
            if i1 is None or i2 is None:
                errors.append(f"{at}: parameters must be integers, got {p1!r}, {p2!r}")
                continue
            if isinstance(score, bool) or not isinstance(score, numbers.Real):
                errors.append(f"{at}: score must be a number, got {score!r}")
                continue
            if kind == "stream_llm":
                if i1 < 0 or i2 < 0:
                    errors.append(f"{at}: stream_llm n_init/n_local must be >= 0, got {i1}, {i2}")
                    continue
                if i2 == 0:
                    summary.notes.append(f"{at}: stream_llm n_local=0, rows past n_init={i1} "
                                         "attend no key and output 0")
            elif kind == "block_sparse" and i1 < 1:
                summary.notes.append(f"{at}: block_sparse top-k {i1} runs as 1")
            elif kind == "vertical_and_slash" and (i1 < 30 or i2 < 50):
                summary.notes.append(f"{at}: vertical_and_slash sizes ({i1}, {i2}) run as "
                                     f"({max(i1, 30)}, {max(i2, 50)})")
            counts[(kind, i1, i2)] += 1
        if n_heads is not None:
            missing = n_heads - len(named)
            summary.defaulted += missing
            counts[DEFAULT_RECORD[:3]] += missing
    if n_layers is not None and n_heads is not None and len(cfg) < n_layers:
        missing = (n_layers - len(cfg)) * n_heads
        summary.defaulted += missing
        counts[DEFAULT_RECORD[:3]] += missing
    if errors:
        shown = "\n  ".join(errors[:20])
        more = f"\n  ... and {len(errors) - 20} more" if len(errors) > 20 else ""
        raise PatternConfigError(f"{where}: {len(errors)} problem(s):\n  {shown}{more}")
    summary.counts = {k: v for k, v in counts.items() if v}
    return summary

"""Write and check per-head pattern files.

    python -m minference.configs.generate check FILE... [--layers 32 --heads 32]
    python -m minference.configs.generate uniform --kind block_sparse --p1 100 -o OUT
    python -m minference.configs.generate mix \\
        --mix 0.3:stream_llm:128:4096,0.6:block_sparse:100,0.1:dense --seed 0 -o OUT
    python -m minference.configs.generate probe --targets-from BEST.json \\
        [--targets-kind stream_llm] --kind block_sparse --p1 16 -o OUT
    python -m minference.configs.generate layers --ranges 8-13,7-14 --topks 1,2,4 \\
        --out-dir DIR
    python -m minference.configs.generate pathb --targets-from BEST.json --out-dir DIR

``pathb`` writes the reference's probe and sweep file set with its default
arguments (benchmarks/prepare_phi3_pathb_configs.py:189-300); ``probe`` and
``pathb`` take their target heads from an existing pattern file (the heads of
``--targets-kind`` there, with their scores), which for the original Phi-3
best pattern and kind stream_llm are the reference's 43 probe heads.  Every
written file passes ``validate_config``.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
from typing import List, Optional

from . import patterns as P


def _parse_mix(text: str) -> List[tuple]:
    """``frac:type[:p1[:p2]]`` entries, comma-separated."""
    mix = []
    for item in text.split(","):
        if not item.strip():
            continue
        parts = item.strip().split(":")
        if len(parts) < 2 or len(parts) > 4:
            raise ValueError(f"mix entry {item!r} is not frac:type[:p1[:p2]]")
        frac = float(parts[0])
        p = [int(x) for x in parts[2:]] + [0] * (4 - len(parts))
        mix.append((frac, P.record(parts[1], p[0], p[1])))
    if not mix:
        raise ValueError("empty mix")
    return mix


def _emit(path: str, cfg, n_layers: int, n_heads: int, indent: int) -> None:
    s = P.validate_config(cfg, n_layers, n_heads, where=path)
    d = os.path.dirname(os.path.abspath(path))
    os.makedirs(d, exist_ok=True)
    P.write(path, cfg, indent=indent)
    kinds = ", ".join(f"{k} {n}" for k, n in sorted(s.kind_counts().items()))
    print(f"wrote {path}: {kinds}")


def _targets(args) -> list:
    cfg = P.load(args.targets_from, args.layers, args.heads)
    t = P.heads_of(cfg, args.targets_kind)
    if not t:
        raise SystemExit(f"{args.targets_from}: no {args.targets_kind} heads to probe")
    return t


def main(argv: Optional[List[str]] = None) -> int:
    ap = argparse.ArgumentParser(prog="python -m minference.configs.generate",
                                 description=__doc__.split("\n\n")[0])
    ap.add_argument("--layers", type=int, default=P.NUM_LAYERS_PHI3)
    ap.add_argument("--heads", type=int, default=P.NUM_HEADS_PHI3)
    ap.add_argument("--indent", type=int, default=2)
    sub = ap.add_subparsers(dest="cmd", required=True)

    c = sub.add_parser("check", help="validate pattern files and print what they ask for")
    c.add_argument("files", nargs="+")
    c.add_argument("--notes", action="store_true", help="list clamped or empty-window heads")

    u = sub.add_parser("uniform", help="one record for every head")
    m = sub.add_parser("mix", help="seeded fixed-count mix over all layer x head slots")
    m.add_argument("--mix", required=True, help="frac:type[:p1[:p2]],...")
    m.add_argument("--seed", type=int, default=0)
    pr = sub.add_parser("probe", help="target heads sparse, the others dense")
    for q in (u, pr):
        q.add_argument("--kind", required=True, choices=P.KINDS)
        q.add_argument("--p1", type=int, default=0)
        q.add_argument("--p2", type=int, default=0)
    for q in (u, m, pr):
        q.add_argument("-o", "--output", required=True)
    lr = sub.add_parser("layers", help="block_sparse on all heads of layer ranges, others dense")
    lr.add_argument("--ranges", required=True, help='e.g. "8-13,7-14"')
    lr.add_argument("--topks", required=True, help='e.g. "1,2,4"')
    lr.add_argument("--out-dir", required=True)
    pb = sub.add_parser("pathb", help="the reference's default probe and sweep file set")
    pb.add_argument("--out-dir", required=True)
    pb.add_argument("--n-init", type=int, default=128)
    pb.add_argument("--n-local", type=int, default=896)
    pb.add_argument("--topk-blocks", type=int, default=16)
    for q in (pr, pb):
        q.add_argument("--targets-from", required=True, help="pattern file naming the targets")
        q.add_argument("--targets-kind", default="stream_llm", choices=P.KINDS)
    args = ap.parse_args(argv)
    L, H = args.layers, args.heads

    if args.cmd == "check":
        bad = 0
        for f in args.files:
            try:
                with open(f) as fh:
                    s = P.validate_config(json.load(fh), L, H, where=f)
            except (OSError, ValueError) as e:   # PatternConfigError and JSON errors
                print(f"FAIL {e}")
                bad += 1
                continue
            recs = ", ".join(f"{k[0]}({k[1]},{k[2]}) x{n}" for k, n in
                             sorted(s.counts.items(), key=lambda kv: -kv[1]))
            print(f"ok   {f}: {recs}; {s.defaulted} defaulted, {len(s.notes)} notes")
            if args.notes:
                for n in s.notes:
                    print(f"     {n}")
        return 1 if bad else 0
    if args.cmd == "uniform":
        _emit(args.output, P.uniform_config(args.kind, args.p1, args.p2, L, H), L, H, args.indent)
    elif args.cmd == "mix":
        _emit(args.output, P.mixed_config(_parse_mix(args.mix), args.seed, L, H), L, H,
              args.indent)
    elif args.cmd == "probe":
        cfg = P.probe_config(_targets(args), P.record(args.kind, args.p1, args.p2),
                             n_layers=L, n_heads=H)
        _emit(args.output, cfg, L, H, args.indent)
    elif args.cmd == "layers":
        ranges = P.parse_layer_ranges(args.ranges, L)
        topks = P.parse_topks(args.topks)
        if not ranges or not topks:
            raise SystemExit("--ranges and --topks must both name at least one value")
        for lo, hi in ranges:
            for t in topks:
                cfg = P.layer_range_config(range(lo, hi + 1), P.record("block_sparse", t),
                                           n_layers=L, n_heads=H)
                _emit(os.path.join(args.out_dir, P.layer_range_name(lo, hi, t)), cfg, L, H,
                      args.indent)
    elif args.cmd == "pathb":
        if (L, H) != (P.NUM_LAYERS_PHI3, P.NUM_HEADS_PHI3):
            raise SystemExit("pathb writes the 32 x 32 Phi-3 set")
        files = P.pathb_configs(_targets(args), args.n_init, args.n_local, args.topk_blocks)
        for name, cfg in files.items():
            _emit(os.path.join(args.out_dir, name), cfg, L, H, args.indent)
    return 0


if __name__ == "__main__":
    sys.exit(main())

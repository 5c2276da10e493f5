"""Write pattern_configs.json: golden data for the pattern-file tooling.

Reads the reference's pattern files (minference/configs/*.json in the
MInference-NPU checkout, plain JSON data) and records, per file, the SHA-256
of its canonical JSON text and its (type, p1, p2) head counts; for the
original Phi-3 best pattern it also records every head's (type, p1, p2) as a
record table plus a 32 x 32 code matrix, and the scores of its stream_llm
heads (the probe targets of benchmarks/prepare_phi3_pathb_configs.py:49-93).

    python tests/golden/make_pattern_fixtures.py /root/reference/MInference-NPU
"""

from __future__ import annotations

import collections
import glob
import hashlib
import json
import os
import sys

BEST = "Phi_3_mini_128k_instruct_kv_out_v32_fit_o_best_pattern.json"
CODES = "abcdefghijklmnopqrstuvwxyz"


def canonical_sha256(cfg) -> str:
    return hashlib.sha256(json.dumps(cfg).encode()).hexdigest()


def main(root: str) -> None:
    out = {"files": {}, "best_pattern": None}
    for path in sorted(glob.glob(os.path.join(root, "minference", "configs", "*.json"))):
        with open(path) as f:
            cfg = json.load(f)
        counts = collections.Counter(f"{r[0]}:{r[1]}:{r[2]}" for layer in cfg
                                     for r in layer.values())
        out["files"][os.path.basename(path)] = {"sha256": canonical_sha256(cfg),
                                                "counts": dict(sorted(counts.items()))}
        if os.path.basename(path) == BEST:
            recs = sorted({tuple(r[:3]) for layer in cfg for r in layer.values()})
            code = {r: CODES[i] for i, r in enumerate(recs)}
            out["best_pattern"] = {
                "name": BEST,
                "records": [list(r) for r in recs],
                "codes": ["".join(code[tuple(layer[str(h)][:3])] for h in range(len(layer)))
                          for layer in cfg],
                "stream_scores": [[li, int(h), r[3]] for li, layer in enumerate(cfg)
                                  for h, r in layer.items() if r[0] == "stream_llm"],
            }
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "pattern_configs.json")
    with open(dst, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    print(f"wrote {dst}: {len(out['files'])} files")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/MInference-NPU")

"""Pattern-file tooling (CPU): the probe / sweep generators against the
reference's own pattern files, and the validator.

The golden data (tests/golden/pattern_configs.json, written by
make_pattern_fixtures.py from the reference's minference/configs/*.json)
holds each reference file's canonical SHA-256 and head counts, and the
original Phi-3 best pattern as a record table + code matrix.  Regenerating a
reference file here and hashing it pins the generator's records, scores, key
order, layer count and file names to the reference's output."""

from __future__ import annotations

import copy
import hashlib
import json
import os
import re

import pytest

from minference.configs import generate as G
from minference.configs import patterns as P
from minference.modules import minference_forward as MF

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "pattern_configs.json")


@pytest.fixture(scope="module")
def gold():
    with open(GOLD) as f:
        return json.load(f)


def _sha(cfg) -> str:
    return hashlib.sha256(json.dumps(cfg).encode()).hexdigest()


def _best_pattern(gold):
    """The original best pattern from its code matrix; stream_llm heads carry
    their recorded scores, the others score 1.0 (their scores are not kept)."""
    b = gold["best_pattern"]
    scores = {(l, h): s for l, h, s in b["stream_scores"]}
    cfg = []
    for li, row in enumerate(b["codes"]):
        layer = {}
        for h, c in enumerate(row):
            kind, p1, p2 = b["records"][ord(c) - ord("a")]
            layer[str(h)] = [kind, p1, p2, scores.get((li, h), 1.0)]
        cfg.append(layer)
    return cfg


def _counts(cfg):
    out = {}
    for layer in cfg:
        for r in layer.values():
            key = f"{r[0]}:{r[1]}:{r[2]}"
            out[key] = out.get(key, 0) + 1
    return out


def test_best_pattern_fixture_consistent(gold):
    cfg = _best_pattern(gold)
    assert _counts(cfg) == gold["files"][gold["best_pattern"]["name"]]["counts"]
    s = P.validate_config(cfg)
    assert s.defaulted == 0 and s.kind_counts() == {"vertical_and_slash": 981, "stream_llm": 43}


def test_probe_targets_from_best_pattern(gold):
    t = P.heads_of(_best_pattern(gold), "stream_llm")
    assert len(t) == 43
    assert t == sorted(t)                       # layer-major, head-ascending
    assert {l for l, _, _ in t} == set(range(8, 14))


def _regenerate(name, targets):
    """Generator call for a reference file name; None for the best pattern."""
    pre = P.PATHB_PREFIX
    if name == pre + "stream_llm_aligned_dense_others.json":
        return P.probe_config(targets, P.record("stream_llm", 128, 896))
    m = re.fullmatch(re.escape(pre) + r"block_sparse_probe_dense_others(?:_topk(\d+))?\.json", name)
    if m:
        return P.probe_config(targets, P.record("block_sparse", int(m.group(1) or 16)))
    m = re.fullmatch(re.escape(pre) + r"block_sparse_all_heads(?:_topk(\d+))?_latency\.json", name)
    if m:
        return P.uniform_config("block_sparse", int(m.group(1) or 16))
    m = re.fullmatch(re.escape(pre) + r"block_sparse_layers(\d+)_(\d+)_all_heads_topk(\d+)_latency\.json",
                     name)
    if m:
        lo, hi, k = (int(g) for g in m.groups())
        assert P.layer_range_name(lo, hi, k) == name
        return P.layer_range_config(range(lo, hi + 1), P.record("block_sparse", k))
    return None


def test_every_reference_file_regenerates_bit_exact(gold):
    targets = P.heads_of(_best_pattern(gold), "stream_llm")
    done = 0
    for name, info in gold["files"].items():
        cfg = _regenerate(name, targets)
        if cfg is None:
            assert name == gold["best_pattern"]["name"]
            continue
        assert _sha(cfg) == info["sha256"], name
        assert _counts(cfg) == info["counts"], name
        P.validate_config(cfg)
        done += 1
    assert done == len(gold["files"]) - 1 == 30


def test_pathb_default_set_matches_reference(gold, tmp_path):
    """The CLI's pathb set = the reference script's default outputs
    (prepare_phi3_pathb_configs.py:213-300), file names and contents."""
    best = tmp_path / "best.json"
    P.write(str(best), _best_pattern(gold))
    out = tmp_path / "out"
    assert G.main(["pathb", "--targets-from", str(best), "--out-dir", str(out)]) == 0
    names = sorted(os.listdir(out))
    assert len(names) == 9
    for n in names:
        with open(out / n) as f:
            assert _sha(json.load(f)) == gold["files"][n]["sha256"], n


def test_cli_layers_probe_uniform_mix_check(gold, tmp_path, capsys):
    best = tmp_path / "best.json"
    P.write(str(best), _best_pattern(gold))
    assert G.main(["layers", "--ranges", "7-14,9-12", "--topks", "1,4", "--out-dir",
                   str(tmp_path / "lr")]) == 0
    for n in os.listdir(tmp_path / "lr"):
        with open(tmp_path / "lr" / n) as f:
            assert _sha(json.load(f)) == gold["files"][n]["sha256"], n
    assert len(os.listdir(tmp_path / "lr")) == 4
    pr = tmp_path / "probe.json"
    assert G.main(["probe", "--targets-from", str(best), "--kind", "block_sparse", "--p1", "2",
                   "-o", str(pr)]) == 0
    with open(pr) as f:
        assert _sha(json.load(f)) == gold["files"][P.PATHB_PREFIX +
                                                   "block_sparse_probe_dense_others_topk2.json"]["sha256"]
    un = tmp_path / "uni.json"
    assert G.main(["uniform", "--kind", "block_sparse", "--p1", "4", "-o", str(un)]) == 0
    with open(un) as f:
        assert _sha(json.load(f)) == gold["files"][P.PATHB_PREFIX +
                                                   "block_sparse_all_heads_topk4_latency.json"]["sha256"]
    mx = tmp_path / "mix.json"
    assert G.main(["mix", "--mix", "0.3:stream_llm:128:4096,0.6:block_sparse:100,0.1:dense",
                   "--seed", "3", "-o", str(mx)]) == 0
    s = P.load(str(mx))
    assert s == P.mixed_config([(0.3, P.record("stream_llm", 128, 4096)),
                                (0.6, P.record("block_sparse", 100)), (0.1, P.record("dense"))], 3)
    assert P.validate_config(s).kind_counts() == {"stream_llm": 307, "block_sparse": 614, "dense": 103}
    bad = tmp_path / "bad.json"
    bad.write_text(json.dumps([{"0": ["sparse", 1, 0, 1.0]}]))
    capsys.readouterr()
    assert G.main(["check", str(mx), str(bad), str(best)]) == 1
    text = capsys.readouterr().out
    assert text.count("ok   ") == 2 and "FAIL" in text and "'sparse'" in text


def test_baseline_mixes():
    """BASELINE configs 4 and 5: 1024 heads 30/60/10 stream(128,4096) /
    block(100) / dense, and 50/50 stream(128,8192) / block(160)."""
    c4 = P.mixed_config([(0.3, P.record("stream_llm", 128, 4096)),
                         (0.6, P.record("block_sparse", 100)), (0.1, P.record("dense"))])
    c5 = P.mixed_config([(0.5, P.record("stream_llm", 128, 8192)),
                         (0.5, P.record("block_sparse", 160))])
    assert P.validate_config(c4).counts == {("stream_llm", 128, 4096): 307,
                                            ("block_sparse", 100, 0): 614, ("dense", 0, 0): 103}
    assert P.validate_config(c5).kind_counts() == {"stream_llm": 512, "block_sparse": 512}


def test_parsers():
    assert P.parse_layer_range("8-13") == (8, 13)
    assert P.parse_layer_range(" 8 ") == (8, 8)
    assert P.parse_layer_ranges("7-14, 8-12,,9") == [(7, 14), (8, 12), (9, 9)]
    for bad in ("13-8", "0-32", "-1", "a-b", "", "3-"):
        with pytest.raises(ValueError):
            P.parse_layer_range(bad)
    assert P.parse_layer_range("0-39", n_layers=40) == (0, 39)
    assert P.parse_topks("1, 2,4,") == [1, 2, 4]
    with pytest.raises(ValueError):
        P.parse_topks("1,0")
    with pytest.raises(ValueError):
        P.probe_config([(32, 0)], P.record("dense"))
    with pytest.raises(ValueError):
        P.layer_range_config([40], P.record("dense"))
    with pytest.raises(ValueError):
        P.pathb_configs([], n_init=100)


# ---------------------------------------------------------------------------
# validator
# ---------------------------------------------------------------------------
def _layer(**over):
    layer = {str(h): P.record("dense") for h in range(32)}
    layer.update(over)
    return layer


@pytest.mark.parametrize("cfg,needle", [
    ({"0": {}}, "top level must be a list"),
    ([[]], "layer 0: expected a dict"),
    ([{"x": ["dense", 0, 0, 1.0]}], "decimal head number"),
    ([{"-1": ["dense", 0, 0, 1.0]}], "decimal head number"),
    ([{"32": ["dense", 0, 0, 1.0]}], "head 32 >= 32 heads"),
    ([{"1": ["dense", 0, 0, 1.0], "01": ["dense", 0, 0, 1.0]}], "named twice"),
    ([{"0": ["dense", 0, 0]}], "record must be [type, p1, p2, score]"),
    ([{"0": "dense"}], "record must be"),
    ([{"0": ["Dense", 0, 0, 1.0]}], "unknown pattern type 'Dense'"),
    ([{"0": ["block_sparse", "100", 0, 1.0]}], "parameters must be integers"),
    ([{"0": ["block_sparse", 1.5, 0, 1.0]}], "parameters must be integers"),
    ([{"0": ["block_sparse", True, 0, 1.0]}], "parameters must be integers"),
    ([{"0": ["dense", 0, 0, "high"]}], "score must be a number"),
    ([{"0": ["dense", 0, 0, None]}], "score must be a number"),
    ([{"0": ["stream_llm", -64, 896, 1.0]}], "n_init/n_local must be >= 0"),
    ([_layer()] * 33, "33 layers, the model has 32"),
])
def test_validator_rejects(cfg, needle):
    with pytest.raises(P.PatternConfigError) as e:
        P.validate_config(cfg, where="x.json")
    assert needle in str(e.value) and str(e.value).startswith("x.json:")


def test_validator_reports_every_problem_with_position():
    cfg = [_layer(), _layer(**{"3": ["sparse", 0, 0, 1.0], "7": ["dense", 0, 0]})]
    with pytest.raises(P.PatternConfigError) as e:
        P.validate_config(cfg)
    msg = str(e.value)
    assert "2 problem(s)" in msg and "layer 1 head '3'" in msg and "layer 1 head '7'" in msg


def test_validator_defaults_and_notes():
    cfg = [_layer(**{"0": ["block_sparse", 0, 0, 1.0], "1": ["vertical_and_slash", 10, 60, 1],
                     "2": ["stream_llm", 64, 0, 1.0], "3": ["block_sparse", 16.0, 0, 1]}),
           {"5": ["stream_llm", 128, 896, 0.5]}]
    s = P.validate_config(cfg)
    assert s.defaulted == 31 + 30 * 32
    assert s.counts[("vertical_and_slash", 1000, 6096)] == s.defaulted
    assert s.counts[("block_sparse", 16, 0)] == 1 and s.counts[("dense", 0, 0)] == 28
    assert len(s.notes) == 3
    assert any("top-k 0 runs as 1" in n for n in s.notes)
    assert any("(10, 60) run as (30, 60)" in n for n in s.notes)
    assert any("n_local=0" in n for n in s.notes)
    # no model shape: only the structure is checked
    assert P.validate_config([{"40": ["dense", 0, 0, 1.0]}] * 40, None, None).defaulted == 0


def test_validated_file_drives_the_dispatcher(gold, tmp_path):
    """A file the validator accepts loads into per-layer plans whose kinds
    match the validator's counts (the dispatcher reads the same file)."""
    path = tmp_path / "best.json"
    cfg = _best_pattern(gold)
    P.write(str(path), cfg)
    s = P.load(str(path))
    assert s == cfg
    kinds = {}
    for layer in range(32):
        plan = MF.build_layer_plan(MF.load_layer_patterns(str(path), layer), 32, 96, 65536, layer)
        for kind, *_ in plan.heads:
            kinds[kind] = kinds.get(kind, 0) + 1
    from minference import _abi
    assert kinds == {_abi.MSA_KIND_VS: 981, _abi.MSA_KIND_STREAM: 43}
    bad = copy.deepcopy(cfg)
    bad[4]["9"] = ["sparse", 0, 0, 1.0]
    P.write(str(path), bad)
    with pytest.raises(P.PatternConfigError):
        P.load(str(path))
    with pytest.raises(ValueError):                 # the dispatcher's own error
        MF.build_layer_plan(MF.load_layer_patterns(str(path), 4), 32, 96, 65536, 4)

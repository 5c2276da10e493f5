"""Model name -> pattern file registry (reference minference/configs/model2path.py:16-20).

``microsoft/Phi-3-mini-128k-instruct`` maps to the same pattern the reference
registers for it: stream_llm(128, 896) on the 43 probe heads of the original
Phi-3 best pattern and dense on the other 981 heads
(``Phi_3_mini_128k_instruct_pathb_stream_llm_aligned_dense_others.json``).
The file in this directory is written by ``patterns.pathb_configs`` from the
probe table below and is identical in content to the reference's file.

``NAMED_CONFIGS`` holds this build's benchmark mixes, which no model name
selects: pass their path as ``config_path``.
"""

from __future__ import annotations

import os

BASE_DIR = os.path.dirname(os.path.abspath(__file__))

# (layer, head, score) of the stream_llm heads of the original Phi-3 best
# pattern: the probe targets of benchmarks/prepare_phi3_pathb_configs.py:49-93.
# Data, not code: the default pattern must name exactly these heads.
PHI3_PROBE_HEADS = (
    (8, 1, 0.96484375), (8, 8, 0.9921875), (8, 10, 0.97265625), (8, 23, 0.98828125),
    (9, 0, 0.984375), (9, 11, 0.94921875), (9, 12, 0.59375), (9, 15, 0.9765625),
    (9, 17, 0.859375), (9, 18, 0.93359375), (9, 20, 0.96875), (9, 21, 0.9296875),
    (9, 31, 0.91796875), (10, 3, 0.984375), (10, 5, 0.62109375), (10, 7, 0.578125),
    (10, 9, 0.8671875), (10, 10, 0.98828125), (10, 11, 0.80078125), (10, 15, 1.0),
    (10, 16, 0.93359375), (10, 18, 0.96875), (10, 21, 0.94921875), (10, 22, 0.91796875),
    (10, 25, 0.953125), (10, 28, 0.98046875), (11, 6, 0.8046875), (11, 7, 0.9921875),
    (11, 10, 0.65234375), (11, 12, 0.69140625), (11, 20, 0.85546875), (11, 23, 0.99609375),
    (11, 25, 0.93359375), (11, 29, 0.59765625), (11, 30, 0.98046875), (12, 12, 0.82421875),
    (12, 16, 0.83203125), (12, 20, 0.84765625), (12, 25, 0.984375), (12, 26, 0.8125),
    (13, 5, 0.98828125), (13, 25, 0.9921875), (13, 27, 0.921875),
)

PHI3_DEFAULT_NAME = "Phi_3_mini_128k_instruct_pathb_stream_llm_aligned_dense_others.json"
PHI3_DEFAULT = os.path.join(BASE_DIR, PHI3_DEFAULT_NAME)

# All 1024 heads sparse: half stream_llm(128, 4096), half block_sparse(top-100),
# seeded assignment (patterns.headline_config(seed=0)); the bench's 64K mix.
PHI3_HEADLINE = os.path.join(BASE_DIR, "Phi_3_mini_128k_instruct_stream_block_50_50.json")

MODEL2PATH = {
    "microsoft/Phi-3-mini-128k-instruct": PHI3_DEFAULT,
}

NAMED_CONFIGS = {
    "phi3_stream_block_50_50": PHI3_HEADLINE,
}


def default_phi3_config():
    """The registered Phi-3 pattern, built from the probe table."""
    from .patterns import pathb_configs

    return pathb_configs(PHI3_PROBE_HEADS)[PHI3_DEFAULT_NAME]


def get_support_models():
    return list(MODEL2PATH.keys())

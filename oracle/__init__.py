"""CPU oracle for the sparse prefill attention path (test infrastructure only).

This package restates the reference algorithms (white-jim/MInference-NPU) in
numpy so that tests can check the HIP kernels against them.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it; the product (``minference-npu_amd/``) never does.
"""

from .msa_oracle import *  # noqa: F401,F403

"""Import-path alias of ``minference.ops.streaming_kernel`` for code written
against the reference module name (ops/streaming_kernel_npu.py)."""

from .streaming_kernel import streaming_forward

__all__ = ["streaming_forward"]

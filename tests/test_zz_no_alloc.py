"""The no-allocation decode entry point (msa_decode_attention_noalloc)
against the workspace entry point it mirrors (msa_decode_attention), both
called through the C ABI: two calls in a row, the second smaller, each
bit-identical to the workspace call (same kernels, same splits) and within
2e-3 of the oracle (reference backend_npu/attention.py:274-314)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("order", ["large_then_small"])
def test_decode_noalloc_matches_workspace_entry(gpu_device, order):
    from minference import _abi

    cases = [(2, 32, 8, 70000, 128, torch.bfloat16), (1, 4, 4, 1000, 96, torch.float16)]
    for B, H, H_kv, S, D, dtype in cases:
        print(f"[noalloc] B={B} H={H} H_kv={H_kv} S={S} D={D} {dtype}", flush=True)
        assert _abi.decode_workspace_bytes(B, H, S, D) <= _abi.MSA_DECODE_SCRATCH_BYTES
        g = torch.Generator(device=gpu_device).manual_seed(S)
        q = torch.randn(B, H, 1, D, generator=g, device=gpu_device).to(dtype)
        k = torch.randn(B, H_kv, S, D, generator=g, device=gpu_device).to(dtype)
        v = torch.randn(B, H_kv, S, D, generator=g, device=gpu_device).to(dtype)
        scale = D ** -0.5
        ref_out = torch.empty(B, H, 1, D, dtype=torch.float32, device=gpu_device)
        out = torch.full_like(ref_out, float("nan"))
        _abi.decode_attention(q, k, v, ref_out, scale)
        _abi.decode_attention_noalloc(q, k, v, out, scale)
        torch.cuda.synchronize()
        assert torch.equal(out, ref_out)
        rep = H // H_kv
        kn = np.repeat(k.float().cpu().numpy(), rep, 1)
        vn = np.repeat(v.float().cpu().numpy(), rep, 1)
        ref = O.dense_causal(q.float().cpu().numpy(), kn, vn, scale=scale)
        err = np.abs(out.cpu().numpy() - ref).max()
        assert err < 2e-3, err
        # q-dtype output as well
        o16 = torch.empty(B, H, 1, D, dtype=dtype, device=gpu_device)
        r16 = torch.empty_like(o16)
        _abi.decode_attention(q, k, v, r16, scale)
        _abi.decode_attention_noalloc(q, k, v, o16, scale)
        torch.cuda.synchronize()
        assert torch.equal(o16, r16)

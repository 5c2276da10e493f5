"""msa_rope_qk on the GPU: bit-exact with HF's eager apply_rotary_pos_emb
(run by torch on the same device) and with the oracle, over full and partial
rotary, GQA, fp16, per-batch and broadcast tables, views of a fused qkv
projection rotated in place, and inside the patched Phi-3 forward."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from msa_data import dtype_tag
from test_rope import hf_rope, rope_tables

pytestmark = pytest.mark.gpu

CASES = [
    # (B, H, H_kv, S, D, rot, dtype, random_halves, table_batch)
    (1, 32, 32, 1000, 96, 96, torch.bfloat16, False, 1),
    (2, 8, 2, 777, 96, 96, torch.bfloat16, True, 2),
    (2, 4, 4, 300, 96, 96, torch.bfloat16, True, 1),     # one table broadcast over the batch
    (1, 6, 2, 513, 128, 96, torch.bfloat16, True, 1),    # partial rotary
    (1, 4, 4, 400, 64, 64, torch.float16, True, 1),
    (1, 4, 1, 257, 128, 128, torch.float16, False, 1),
    (1, 2, 2, 1, 96, 96, torch.bfloat16, True, 1),       # one token (decode step)
]


def _ids(c):
    return f"{c[:6]}{dtype_tag(c[6])}{'-rand' if c[7] else ''}-tb{c[8]}"


@pytest.mark.parametrize("case", CASES, ids=[_ids(c) for c in CASES])
def test_rope_bit_exact_vs_hf_and_oracle(gpu_device, case):
    from minference.ops.rope import apply_rotary_pos_emb

    B, H, Hkv, S, D, rot, dtype, rnd, tb = case
    print(f"[rope] case {case}", flush=True)
    g = torch.Generator().manual_seed(S * 7 + D)
    q = (torch.randn(B, H, S, D, generator=g) * 3).to(dtype)
    k = (torch.randn(B, Hkv, S, D, generator=g) * 3).to(dtype)
    cos, sin = rope_tables(tb, S, rot, dtype, offset=4000, random_halves=rnd, seed=S)
    dq, dk, dc, ds = (t.to(gpu_device) for t in (q, k, cos, sin))
    gq, gk = apply_rotary_pos_emb(dq, dk, dc, ds)
    torch.cuda.synchronize()
    rq, rk = hf_rope(dq, dk, dc, ds)                   # eager HF on the same GPU
    assert torch.equal(gq, rq) and torch.equal(gk, rk)
    tag = dtype_tag(dtype)
    cn, sn = cos.float().numpy(), sin.float().numpy()
    assert np.array_equal(gq.float().cpu().numpy(), O.rope_rotate_half(q.float().numpy(), cn, sn, tag))
    assert np.array_equal(gk.float().cpu().numpy(), O.rope_rotate_half(k.float().numpy(), cn, sn, tag))
    # the inputs are untouched and the outputs sit in [B, S, H, D] memory
    assert torch.equal(dq.cpu(), q)
    assert gq.transpose(1, 2).is_contiguous()


@pytest.mark.parametrize("n_kv", [32, 8])
def test_rope_in_place_on_fused_qkv_views(gpu_device, n_kv):
    """The patched forward's case: q and k are views of one qkv projection
    output [B, S, (H + 2 H_kv) D]; they are rotated in place and v stays."""
    from minference.ops.rope import apply_rotary_pos_emb

    B, H, S, D = 1, 32, 2048 + 5, 96
    g = torch.Generator(device=gpu_device).manual_seed(3)
    qkv = torch.randn(B, S, (H + 2 * n_kv) * D, generator=g, device=gpu_device).to(torch.bfloat16)
    ref = qkv.clone()
    q = qkv[..., :H * D].view(B, S, H, D).transpose(1, 2)
    k = qkv[..., H * D:(H + n_kv) * D].view(B, S, n_kv, D).transpose(1, 2)
    cos, sin = (t.to(gpu_device) for t in rope_tables(B, S, D, torch.bfloat16, offset=17))
    rq, rk = hf_rope(ref[..., :H * D].view(B, S, H, D).transpose(1, 2),
                     ref[..., H * D:(H + n_kv) * D].view(B, S, n_kv, D).transpose(1, 2), cos, sin)
    oq, ok = apply_rotary_pos_emb(q, k, cos, sin, inplace=True)
    torch.cuda.synchronize()
    assert oq.data_ptr() == q.data_ptr() and ok.data_ptr() == k.data_ptr()
    assert torch.equal(q, rq) and torch.equal(k, rk)
    assert torch.equal(qkv[..., (H + n_kv) * D:], ref[..., (H + n_kv) * D:])


def test_rope_64k_matches_hf(gpu_device):
    """BASELINE shape (32 heads x 96, 64K tokens): bit-exact with eager HF."""
    from minference.ops.rope import apply_rotary_pos_emb

    B, H, S, D = 1, 32, 65536, 96
    g = torch.Generator(device=gpu_device).manual_seed(0)
    q = torch.randn(B, S, H, D, generator=g, device=gpu_device).to(torch.bfloat16).transpose(1, 2)
    k = torch.randn(B, S, H, D, generator=g, device=gpu_device).to(torch.bfloat16).transpose(1, 2)
    cos, sin = (t.to(gpu_device) for t in rope_tables(B, S, D, torch.bfloat16))
    gq, gk = apply_rotary_pos_emb(q, k, cos, sin)
    rq, rk = hf_rope(q, k, cos, sin)
    assert torch.equal(gq, rq) and torch.equal(gk, rk)


def test_rope_rejects_what_it_cannot_take(gpu_device):
    from minference import _abi
    from minference.ops.rope import apply_rotary_pos_emb, rope_supported

    q = torch.zeros(1, 2, 8, 96, dtype=torch.bfloat16, device=gpu_device)
    cos = torch.zeros(1, 8, 40, dtype=torch.bfloat16, device=gpu_device)  # rot % 16 != 0
    assert not rope_supported(q, q, cos, cos)
    with pytest.raises(NotImplementedError):
        apply_rotary_pos_emb(q, q, cos, cos)
    c32 = torch.zeros(1, 8, 96, dtype=torch.float32, device=gpu_device)
    assert not rope_supported(q, q, c32, c32)
    c_bad = torch.zeros(1, 1, 8, 96, dtype=torch.bfloat16, device=gpu_device)
    with pytest.raises(ValueError):                  # library validation: S mismatch
        _abi.rope_qk(q, q, c_bad[:, :, :4], c_bad[:, :, :4], q, q)


def test_patched_forward_rope_matches_hf(gpu_device):
    """The patched Phi-3 attention rotates q/k with the HIP kernel in place;
    with the model's own (LongRoPE-scaled) tables the result is the eager HF
    rotation bit for bit."""
    from transformers import Phi3Config, Phi3ForCausalLM

    from minference.modules import minference_forward as MF

    torch.manual_seed(0)
    cfg = Phi3Config(hidden_size=96 * 8, intermediate_size=256, num_hidden_layers=1,
                     num_attention_heads=8, num_key_value_heads=8, vocab_size=128,
                     max_position_embeddings=131072, original_max_position_embeddings=4096,
                     rope_scaling={"type": "longrope", "short_factor": [1.05] * 48,
                                   "long_factor": [1.3] * 48},
                     pad_token_id=0, bos_token_id=1, eos_token_id=2)
    model = Phi3ForCausalLM(cfg).to(device=gpu_device, dtype=torch.bfloat16).eval()
    attn = model.model.layers[0].self_attn
    S = 5000                                            # past the original 4096: long factors
    x = torch.randn(1, S, 96 * 8, device=gpu_device).to(torch.bfloat16)
    pos = torch.arange(S, device=gpu_device)[None]
    cos, sin = model.model.rotary_emb(x, pos)
    with torch.no_grad():
        qkv = attn.qkv_proj(x)
    q = qkv[..., :768].view(1, S, 8, 96).transpose(1, 2)
    k = qkv[..., 768:1536].view(1, S, 8, 96).transpose(1, 2)
    rq, rk = hf_rope(q.clone(), k.clone(), cos, sin)
    gq, gk = MF._apply_rope(attn, q, k, cos, sin)
    torch.cuda.synchronize()
    assert gq.data_ptr() == q.data_ptr()               # the HIP path ran, in place
    assert torch.equal(gq, rq) and torch.equal(gk, rk)

"""oracle.rope_rotate_half pinned on the CPU (no GPU needed).

Against HF Phi-3's apply_rotary_pos_emb run by CPU torch in bf16 / fp16 (the
function the reference's forward looks up and calls,
minference/modules/minference_forward.py:205-212, 336-341), bit for bit, with
real position tables and with random tables whose two halves differ (real
tables repeat cos[i] == cos[i + rot/2], which would hide a swapped half);
and, in fp64, against the rotation it is: each (i, i + rot/2) pair turned by
its angle, norms kept."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from msa_data import dtype_tag


def hf_rope(q, k, cos, sin):
    from transformers.models.phi3.modeling_phi3 import apply_rotary_pos_emb

    return apply_rotary_pos_emb(q, k, cos, sin)


def rope_tables(B, S, rot, dtype, theta=10000.0, offset=0, random_halves=False, seed=0):
    """[B, S, rot] cos/sin as HF builds them (cat(freqs, freqs), cast to the
    model dtype), or random values in [-1, 1] with independent halves."""
    if random_halves:
        g = torch.Generator().manual_seed(seed)
        c = torch.rand(B, S, rot, generator=g) * 2 - 1
        s = torch.rand(B, S, rot, generator=g) * 2 - 1
        return c.to(dtype), s.to(dtype)
    inv = 1.0 / (theta ** (torch.arange(0, rot, 2, dtype=torch.float32) / rot))
    pos = torch.arange(offset, offset + S, dtype=torch.float32)
    f = pos[:, None] * inv[None, :]
    emb = torch.cat([f, f], dim=-1)[None].expand(B, S, rot)
    return emb.cos().to(dtype), emb.sin().to(dtype)


CASES = [
    # (B, H, H_kv, S, D, rot, dtype, random_halves)
    (1, 4, 4, 97, 96, 96, torch.bfloat16, False),
    (2, 4, 2, 64, 96, 96, torch.bfloat16, True),
    (1, 3, 1, 50, 128, 96, torch.bfloat16, True),    # partial rotary
    (1, 2, 2, 33, 64, 64, torch.float16, True),
    (1, 2, 1, 70, 128, 128, torch.float16, False),
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[:6]}{dtype_tag(c[6])}{'-rand' if c[7] else ''}"
                                             for c in CASES])
def test_rope_oracle_matches_hf_bitwise(case):
    B, H, Hkv, S, D, rot, dtype, rnd = case
    g = torch.Generator().manual_seed(S + D)
    q = (torch.randn(B, H, S, D, generator=g) * 3).to(dtype)
    k = (torch.randn(B, Hkv, S, D, generator=g) * 3).to(dtype)
    cos, sin = rope_tables(B, S, rot, dtype, offset=1000, random_halves=rnd, seed=S)
    rq, rk = hf_rope(q, k, cos, sin)
    tag = dtype_tag(dtype)
    oq = O.rope_rotate_half(q.float().numpy(), cos.float().numpy(), sin.float().numpy(), tag)
    ok = O.rope_rotate_half(k.float().numpy(), cos.float().numpy(), sin.float().numpy(), tag)
    assert np.array_equal(oq, rq.float().numpy())
    assert np.array_equal(ok, rk.float().numpy())


def test_rope_oracle_is_a_rotation():
    """Without 16-bit rounding (dtype "fp32"): pair (x_i, x_{i+h}) is turned
    by the angle whose cos/sin the table holds (checked in complex fp64),
    norms are kept and the pass-through dims are untouched."""
    B, H, S, D, rot = 1, 2, 40, 128, 96
    rng = np.random.default_rng(1)
    x = rng.standard_normal((B, H, S, D)).astype(np.float32).astype(np.float64)
    ang = rng.uniform(-np.pi, np.pi, (B, S, rot // 2))
    cos = np.concatenate([np.cos(ang), np.cos(ang)], -1)
    sin = np.concatenate([np.sin(ang), np.sin(ang)], -1)
    out = O.rope_rotate_half(x, cos, sin, "fp32").astype(np.float64)
    h = rot // 2
    z = x[..., :h] + 1j * x[..., h:rot]
    want = z * np.exp(1j * ang)[:, None]
    assert np.allclose(out[..., :h], want.real, atol=1e-5)
    assert np.allclose(out[..., h:rot], want.imag, atol=1e-5)
    assert np.allclose(np.abs(z), np.hypot(out[..., :h], out[..., h:rot]), atol=1e-5)
    assert np.array_equal(out[..., rot:], x[..., rot:])


def test_rope_oracle_catches_planted_mistakes():
    """A swapped half, a wrong sign or a fused (unrounded) product each fail
    the HF comparison above on random-halves tables."""
    B, H, S, D = 1, 2, 31, 96
    g = torch.Generator().manual_seed(5)
    q = (torch.randn(B, H, S, D, generator=g) * 3).to(torch.bfloat16)
    cos, sin = rope_tables(B, S, D, torch.bfloat16, random_halves=True, seed=2)
    rq, _ = hf_rope(q, q, cos, sin)
    want = rq.float().numpy()
    xn, cn, sn = q.float().numpy(), cos.float().numpy(), sin.float().numpy()
    good = O.rope_rotate_half(xn, cn, sn, "bf16")
    assert np.array_equal(good, want)
    swapped = O.rope_rotate_half(xn, np.concatenate([cn[..., 48:], cn[..., :48]], -1), sn, "bf16")
    flipped = O.rope_rotate_half(xn, cn, -sn, "bf16")
    c, s = cn[:, None], sn[:, None]
    x1, x2 = xn[..., :48], xn[..., 48:]
    fused = np.concatenate([O.bf16_round(x1 * c[..., :48] - x2 * s[..., :48]),
                            O.bf16_round(x2 * c[..., 48:] + x1 * s[..., 48:])], -1)
    for bad in (swapped, flipped, fused):
        assert not np.array_equal(bad, want)

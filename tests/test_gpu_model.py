"""Parity inside the full-prefill configurations (BASELINE configs 4 and 5).

A random-init Phi-3-mini-128k-shaped model (hidden 3072, 32 heads x 96, MLP
8192, vocab 32064, LongRoPE tables, bf16), with fewer layers, is prefilled
through the patched forward with the configs' seeded per-head mixes at their
full lengths: 32768 tokens with 30 % stream_llm(128, 4096) / 60 %
block_sparse(top-100) / 10 % dense, and 131072 tokens with 50 % stream_llm(128,
8192) / 50 % block_sparse(top-160).  Every layer launch is captured; on
sampled rows of sampled heads of each kind its output is compared with the
oracle on the very q/k/v the model produced (block ids from the oracle
selector), within the bf16-output bound."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from minference import MInference
from minference import _abi
from minference.configs import patterns as P
from minference.modules import minference_forward as MF

pytestmark = pytest.mark.gpu


def phi3_mini_shaped(dev, layers):
    from transformers import Phi3Config, Phi3ForCausalLM

    cfg = Phi3Config(vocab_size=32064, hidden_size=3072, intermediate_size=8192,
                     num_hidden_layers=layers, num_attention_heads=32, num_key_value_heads=32,
                     max_position_embeddings=131072, original_max_position_embeddings=4096,
                     rope_scaling={"type": "longrope", "short_factor": [1.0] * 48,
                                   "long_factor": [4.0] * 48},
                     pad_token_id=32000, bos_token_id=1, eos_token_id=32000)
    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(dev):
            torch.manual_seed(0)
            model = Phi3ForCausalLM(cfg)
    finally:
        torch.set_default_dtype(old)
    return model.eval()


def sample_rows(S, extra=()):
    base = {0, 1, 63, 64, 127, 128, 129, 4095, 4096, 4097, 4224, 8191, 8192, 8320,
            S // 3, S // 2 + 17, S - 65, S - 64, S - 1}
    return sorted(r for r in base.union(extra) if 0 <= r < S)


def row_oracle(qh, kh, vh, rows, vis, scale):
    out = []
    for r in rows:
        js = vis(r)
        lg = kh[js] @ qh[r] * scale
        p = np.exp(lg - lg.max())
        out.append((p / p.sum()) @ vh[js])
    return np.stack(out)


def check_layer(q, k, v, plan, got, per_kind=3):
    S = q.shape[2]
    rows = sample_rows(S)
    by_kind = {}
    for h, hd in enumerate(plan.heads):
        by_kind.setdefault(hd[0], []).append(h)
    for kind, heads in by_kind.items():
        for h in heads[:: max(1, len(heads) // per_kind)][:per_kind]:
            kind_, p1, p2, slot, scale = plan.heads[h]
            qh, kh, vh = (t[0, h].double().cpu().numpy() for t in (q, k, v))
            if kind == _abi.MSA_KIND_STREAM:
                def vis(r, p1=p1, p2=p2):
                    return np.union1d(np.arange(min(p1, r + 1)), np.arange(max(0, r - p2 + 1), r + 1))
            elif kind == _abi.MSA_KIND_BLOCK:
                idx, cnt = O.select_block_sparse_topk_indices(
                    q[:, h:h + 1].float().cpu().numpy(), k[:, h:h + 1].float().cpu().numpy(),
                    p1, "bf16", scale)

                def vis(r, idx=idx, cnt=cnt):
                    bq = r // 64
                    ids = idx[0, 0, bq, :cnt[0, 0, bq]]
                    js = np.concatenate([np.arange(64 * b, 64 * b + 64) for b in ids])
                    return js[js <= r]
            else:
                def vis(r):
                    return np.arange(r + 1)
            ref = row_oracle(qh, kh, vh, rows, vis, scale)
            g = got[0, h, rows].double().cpu().numpy()
            bound = 2e-3 + np.abs(ref) * 2.0 ** -8   # bf16 output of the model
            err = np.abs(g - ref)
            assert (err <= bound).all(), (kind, h, float(err.max()))


@pytest.mark.parametrize("S,layers,mix", [
    (32768, 2, [(0.3, P.record("stream_llm", 128, 4096)), (0.6, P.record("block_sparse", 100)),
                (0.1, P.record("dense"))]),
    (131072, 1, [(0.5, P.record("stream_llm", 128, 8192)), (0.5, P.record("block_sparse", 160))]),
], ids=["cfg4-32k", "cfg5-128k"])
def test_full_prefill_layers_match_oracle(gpu_device, tmp_path, monkeypatch, S, layers, mix):
    print(f"[model] S={S} layers={layers}", flush=True)
    model = phi3_mini_shaped(gpu_device, layers)
    path = tmp_path / "mix.json"
    P.write(str(path), P.mixed_config(mix, seed=0, n_layers=layers))
    captured = []
    real = MF.run_layer_attention

    def spy(q, k, v, plan, out):
        res = real(q, k, v, plan, out)
        captured.append((q.clone(), k.clone(), v.clone(), plan, res.clone()))
        return res

    monkeypatch.setattr(MF, "run_layer_attention", spy)
    patched = MInference(attn_type="minference", config_path=str(path))(model)
    ids = torch.randint(3, 32000, (1, S), device=gpu_device,
                        generator=torch.Generator(device=gpu_device).manual_seed(S))
    with torch.no_grad():
        logits = patched(input_ids=ids, use_cache=True, logits_to_keep=1).logits
    assert torch.isfinite(logits).all()
    assert len(captured) == layers
    del model, patched
    for li, (q, k, v, plan, got) in enumerate(captured):
        print(f"[model] layer {li}: checking sampled rows", flush=True)
        assert not plan.all_dense
        check_layer(q, k, v, plan, got)

"""Parity inside the full-prefill configurations (BASELINE configs 4 and 5).

A random-init Phi-3-mini-128k-shaped model (hidden 3072, 32 heads x 96, MLP
8192, vocab 32064, LongRoPE tables, bf16), with fewer layers, is prefilled
through the patched forward with the configs' seeded per-head mixes at their
full lengths: 32768 tokens with 30 % stream_llm(128, 4096) / 60 %
block_sparse(top-100) / 10 % dense, and 131072 tokens with 50 % stream_llm(128,
8192) / 50 % block_sparse(top-160).  Every layer launch is captured; on one
row in every query block of every head (plus boundary rows) its output is
compared with the oracle's fp64 rows on the very q/k/v the model produced
(block ids from the oracle selector), within the bf16-output bound."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
import row_sampling as RS
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


def sample_rows(S):
    return {0, 1, 63, 64, 127, 128, 129, 4095, 4096, 4097, 4224, 8191, 8192, 8320,
            S // 3, S // 2 + 17, S - 65, S - 64, S - 1}


def check_layer(tag, q, k, v, plan, got):
    """Every head of the layer: one row per query block plus the sampled
    boundary rows, against the oracle's fp64 rows (block ids from the oracle
    selector on that head), within the bf16-output bound."""
    S = q.shape[2]
    qn, kn, vn = (t[0].float().cpu().numpy() for t in (q, k, v))
    gn = got[0].float().cpu().numpy()

    def check(h):
        kind, p1, p2, slot, scale = plan.heads[h]
        ids = cnt = None
        if kind == _abi.MSA_KIND_BLOCK:
            idx, cn = O.select_block_sparse_topk_indices(qn[None, h:h + 1], kn[None, h:h + 1], p1,
                                                         "bf16", scale)
            ids, cnt = idx[0, 0], cn[0, 0]
        rows = RS.block_rows(S, h, extra=sample_rows(S))
        ref = RS.head_rows_reference(qn[h], kn[h], vn[h], rows, kind, p1, p2, scale, ids, cnt)
        err = np.abs(gn[h, rows] - ref)
        bound = 2e-3 + np.abs(ref) * 2.0 ** -8   # bf16 output of the model
        return h, kind, rows.size, float(err.max()), int((err > bound).sum())

    res = RS.map_heads(check, range(q.shape[1]), tag=tag)
    kinds = sorted({r[1] for r in res})
    print(f"{tag} {sum(r[2] for r in res)} rows, kinds {kinds}, worst error "
          f"{max(r[3] for r in res):.3e}", flush=True)
    for h, kind, n, err, n_bad in res:
        assert n_bad == 0, (h, kind, n, err, n_bad)


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
        assert not plan.all_dense
        check_layer(f"[model] S={S} layer {li}:", q, k, v, plan, got)

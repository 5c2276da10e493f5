"""The patched HF Phi-3 forward on the GPU: real kernels inside a model.

A tiny random Phi-3 (head_dim 96) is patched with mixed per-head patterns;
every layer's attention launch is captured and checked against the oracle on
the very inputs the model produced, and a dense-pattern model is compared with
the unpatched HF model end to end."""

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


def _tiny_phi3(device, n_heads=8, n_kv=8, layers=2, seed=0, dtype=torch.bfloat16):
    from transformers import Phi3Config, Phi3ForCausalLM

    torch.manual_seed(seed)
    cfg = Phi3Config(hidden_size=96 * n_heads, intermediate_size=512, num_hidden_layers=layers,
                     num_attention_heads=n_heads, num_key_value_heads=n_kv, vocab_size=256,
                     max_position_embeddings=8192, pad_token_id=0, bos_token_id=1, eos_token_id=2)
    return Phi3ForCausalLM(cfg).to(device=device, dtype=dtype).eval()


def _oracle_layer(q, k, v, plan, tag="bf16"):
    qn, kn, vn = (t.detach().float().cpu().numpy() for t in (q, k, v))
    rep = qn.shape[1] // kn.shape[1]
    kn, vn = np.repeat(kn, rep, 1), np.repeat(vn, rep, 1)
    out = np.zeros(qn.shape)
    for h, (kind, p1, p2, slot, scale) in enumerate(plan.heads):
        sl = slice(h, h + 1)
        if kind == _abi.MSA_KIND_STREAM:
            out[:, sl] = O.streaming_attention(qn[:, sl], kn[:, sl], vn[:, sl], p1, p2, scale=scale)
        elif kind == _abi.MSA_KIND_BLOCK:
            idx, _ = O.select_block_sparse_topk_indices(qn[:, sl], kn[:, sl], p1, tag, scale)
            out[:, sl] = O.block_sparse_from_indices(qn[:, sl], kn[:, sl], vn[:, sl], idx, scale=scale)
        else:
            out[:, sl] = O.dense_causal(qn[:, sl], kn[:, sl], vn[:, sl], scale=scale)
    return out


@pytest.mark.parametrize("n_kv,dtype", [(8, torch.bfloat16), (2, torch.bfloat16), (8, torch.float16)],
                         ids=["kv8-bf16", "kv2-bf16", "kv8-fp16"])
def test_patched_model_layers_match_oracle(gpu_device, tmp_path, monkeypatch, n_kv, dtype):
    model = _tiny_phi3(gpu_device, n_kv=n_kv, dtype=dtype)
    tag = "bf16" if dtype == torch.bfloat16 else "fp16"
    recs = [P.record("stream_llm", 64, 256), P.record("block_sparse", 4), P.record("dense"),
            P.record("block_sparse", 100), P.record("stream_llm", 0, 128), P.record("block_sparse", 1),
            P.record("stream_llm", 128, 512), P.record("dense")]
    path = tmp_path / "mix.json"
    P.write(str(path), [{str(h): recs[(h + layer) % 8] for h in range(8)} for layer in range(2)])
    captured = []
    real = MF.run_layer_attention

    def spy(q, k, v, plan, out):
        res = real(q, k, v, plan, out)
        captured.append((q.clone(), k.clone(), v.clone(), plan, res.float().clone()))
        return res

    monkeypatch.setattr(MF, "run_layer_attention", spy)
    patched = MInference(attn_type="minference", config_path=str(path))(model)
    ids = torch.randint(3, 256, (1, 1000), device=gpu_device,
                        generator=torch.Generator(device=gpu_device).manual_seed(0))
    with torch.no_grad():
        logits = patched(ids).logits
    assert torch.isfinite(logits).all()
    assert len(captured) == 2
    for q, k, v, plan, got in captured:
        assert not plan.all_dense
        assert q.dtype == dtype
        ref = _oracle_layer(q, k, v, plan, tag)
        g = got.cpu().numpy().astype(np.float64)
        # the model's output dtype: one rounding (bf16 2^-8, fp16 2^-11 relative)
        bound = 2e-3 + np.abs(ref) * (2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11)
        assert (np.abs(g - ref) <= bound).all(), np.abs(g - ref).max()


def test_patched_dense_model_matches_hf(gpu_device, tmp_path):
    model = _tiny_phi3(gpu_device)
    ids = torch.randint(3, 256, (1, 700), device=gpu_device,
                        generator=torch.Generator(device=gpu_device).manual_seed(1))
    with torch.no_grad():
        ref = model(ids).logits.float()
    path = tmp_path / "dense.json"
    P.write(str(path), P.uniform_config("dense", n_layers=2, n_heads=8))
    patched = MInference(attn_type="minference", config_path=str(path))(model)
    with torch.no_grad():
        got = patched(ids).logits.float()
        nxt = patched.generate(ids[:, :100], max_new_tokens=3, do_sample=False, use_cache=True)
    assert nxt.shape == (1, 103)
    rel = (got - ref).abs().max() / ref.abs().max()
    assert rel < 2e-2, rel


def test_patched_chunked_prefill_and_decode_match_oracle(gpu_device, tmp_path, monkeypatch):
    """Prefill in two chunks through a cache (the second with S_q < S_k), then
    decode steps: every attention launch of the patched model is checked
    against the oracle on the inputs it received."""
    from transformers import DynamicCache

    model = _tiny_phi3(gpu_device, n_kv=2)
    recs = [P.record("stream_llm", 64, 256), P.record("block_sparse", 3), P.record("dense"),
            P.record("block_sparse", 100)]
    path = tmp_path / "mix.json"
    P.write(str(path), [{str(h): recs[(h + layer) % 4] for h in range(8)} for layer in range(2)])
    captured = []
    real_l, real_d = MF.run_layer_attention, MF.run_decode_attention

    def spy_l(q, k, v, plan, out):
        res = real_l(q, k, v, plan, out)
        captured.append(("layer", q.clone(), k.clone(), v.clone(), plan, res.float().clone()))
        return res

    def spy_d(q, k, v, out, scale):
        res = real_d(q, k, v, out, scale)
        captured.append(("decode", q.clone(), k.clone(), v.clone(), scale, res.float().clone()))
        return res

    monkeypatch.setattr(MF, "run_layer_attention", spy_l)
    monkeypatch.setattr(MF, "run_decode_attention", spy_d)
    patched = MInference(attn_type="minference", config_path=str(path))(model)
    ids = torch.randint(3, 256, (1, 700), device=gpu_device,
                        generator=torch.Generator(device=gpu_device).manual_seed(3))
    cache = DynamicCache()
    with torch.no_grad():
        patched(ids[:, :600], past_key_values=cache, use_cache=True)
        logits = patched(ids[:, 600:], past_key_values=cache, use_cache=True).logits
        nxt = logits[:, -1:].argmax(-1)
        for _ in range(3):
            logits = patched(nxt, past_key_values=cache, use_cache=True).logits
            assert torch.isfinite(logits).all()
            nxt = logits[:, -1:].argmax(-1)
    kinds = [c[0] for c in captured]
    assert kinds == ["layer"] * 4 + ["decode"] * 6, kinds
    assert captured[2][1].shape[2] == 100 and captured[2][2].shape[2] == 700
    assert captured[-1][2].shape[2] == 703
    for kind, q, k, v, plan_or_scale, got in captured:
        if kind == "layer":
            ref = _oracle_layer(q, k, v, plan_or_scale)
        else:
            qn, kn, vn = (t.float().cpu().numpy() for t in (q, k, v))
            rep = qn.shape[1] // kn.shape[1]
            ref = O.dense_causal(qn, np.repeat(kn, rep, 1), np.repeat(vn, rep, 1),
                                 scale=plan_or_scale)
        g = got.cpu().numpy().astype(np.float64)
        bound = 2e-3 + np.abs(ref) * 2.0 ** -8  # bf16 output of the model
        assert (np.abs(g - ref) <= bound).all(), (kind, q.shape, np.abs(g - ref).max())


@pytest.mark.parametrize("n_kv,dtype", [(8, torch.bfloat16), (2, torch.bfloat16), (8, torch.float16)],
                         ids=["kv8-bf16", "kv2-bf16", "kv8-fp16"])
def test_patched_model_vertical_and_slash_heads(gpu_device, tmp_path, monkeypatch, n_kv, dtype):
    """vertical_and_slash heads (explicit records and the default for heads
    missing from the JSON) next to the other kinds; every layer launch is
    checked against the oracle estimator + attention on its own inputs."""
    model = _tiny_phi3(gpu_device, n_kv=n_kv, dtype=dtype)
    tag = "bf16" if dtype == torch.bfloat16 else "fp16"
    layer0 = {"0": P.record("stream_llm", 64, 256), "2": ["vertical_and_slash", 100, 200, 1],
              "3": P.record("block_sparse", 4), "5": P.record("dense"),
              "6": ["vertical_and_slash", 30, 800, 1]}
    layer1 = {str(h): ["vertical_and_slash", 60 + 10 * h, 100 + 50 * h, 1] for h in range(8)}
    path = tmp_path / "vs.json"
    P.write(str(path), [layer0, layer1])
    captured = []
    real = MF.run_layer_attention

    def spy(q, k, v, plan, out):
        res = real(q, k, v, plan, out)
        captured.append((q.clone(), k.clone(), v.clone(), plan, res.float().clone()))
        return res

    monkeypatch.setattr(MF, "run_layer_attention", spy)
    patched = MInference(attn_type="minference", config_path=str(path))(model)
    ids = torch.randint(3, 256, (1, 1500), device=gpu_device,
                        generator=torch.Generator(device=gpu_device).manual_seed(7))
    with torch.no_grad():
        logits = patched(ids).logits
    assert torch.isfinite(logits).all()
    assert len(captured) == 2
    assert captured[0][3].vs_heads == (1, 2, 4, 6, 7)   # 1, 4, 7 default
    for q, k, v, plan, got in captured:
        qn, kn, vn = (t.detach().float().cpu().numpy() for t in (q, k, v))
        rep = qn.shape[1] // kn.shape[1]
        kr, vr = np.repeat(kn, rep, 1), np.repeat(vn, rep, 1)
        ref = _oracle_layer(q, k, v, plan, tag)
        for h, (kind, p1, p2, slot, scale) in enumerate(plan.heads):
            if kind == _abi.MSA_KIND_VS:
                sl = slice(h, h + 1)
                vi, si = O.vs_estimate(qn[:, sl], kr[:, sl], p1, p2, tag)
                ref[:, sl] = O.vertical_slash_from_indices(qn[:, sl], kr[:, sl], vr[:, sl], vi, si,
                                                           scale=scale)
        g = got.cpu().numpy().astype(np.float64)
        # the model's output dtype: one rounding (bf16 2^-8, fp16 2^-11 relative)
        bound = 2e-3 + np.abs(ref) * (2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11)
        assert (np.abs(g - ref) <= bound).all(), np.abs(g - ref).max()

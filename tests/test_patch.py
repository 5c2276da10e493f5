"""Host-side logic of the drop-in surface (CPU): configuration, pattern files,
per-layer plans and the HF patch plumbing.

The plumbing tests swap the device launch (``run_layer_attention``) for a CPU
test double built on the oracle, so the patched forward's own work (QKV
split, RoPE, cache update, output layout, o_proj) is compared with the
unpatched HF model.  The product code itself has no CPU path."""

from __future__ import annotations

import json
import os
import math

import numpy as np
import pytest
import torch

import oracle as O
from minference import MInference, MInferenceConfig, get_support_models, patch_hf
from minference import _abi
from minference.configs import patterns as P
from minference.modules import minference_forward as MF


# ---------------------------------------------------------------------------
# configuration and patterns
# ---------------------------------------------------------------------------
def test_config_semantics(tmp_path):
    cfg = MInferenceConfig(attn_type="minference", model_name="microsoft/Phi-3-mini-128k-instruct")
    assert cfg.config_path.endswith(".json")
    assert cfg.attn_kwargs["starting_layer"] == -1 and cfg.kv_type == "dense"
    assert MInferenceConfig(attn_type="dense").config_path == ""
    assert MInferenceConfig(attn_type="minference_with_dense").attn_type == "dense"
    with pytest.raises(AssertionError):
        MInferenceConfig(attn_type="vllm")
    with pytest.raises(AssertionError):
        MInferenceConfig(attn_type="minference", model_name="unknown/model")
    assert get_support_models() == ["microsoft/Phi-3-mini-128k-instruct"]
    with pytest.raises(ValueError):
        MInference(attn_type="streaming")
    with pytest.raises(NotImplementedError):
        patch_hf(torch.nn.Module(), attn_type="hf")


def test_registered_config_is_reference_default():
    """The Phi-3 name selects the reference's registered pattern
    (minference/configs/model2path.py:16-19): stream_llm(128, 896) on the 43
    probe heads, dense elsewhere; same content as the reference's file
    (hash recorded from it in tests/golden/pattern_configs.json)."""
    import hashlib

    from minference.configs import model2path as M

    path = M.MODEL2PATH["microsoft/Phi-3-mini-128k-instruct"]
    assert os.path.basename(path) == M.PHI3_DEFAULT_NAME
    cfg = json.load(open(path))
    assert len(cfg) == 32 and all(len(layer) == 32 for layer in cfg)
    recs = [tuple(rec[:3]) for layer in cfg for rec in layer.values()]
    assert recs.count(("stream_llm", 128, 896)) == 43 and recs.count(("dense", 0, 0)) == 981
    golden = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                         "pattern_configs.json")))
    sha = hashlib.sha256(json.dumps(cfg).encode()).hexdigest()
    assert sha == golden["files"][M.PHI3_DEFAULT_NAME]["sha256"]
    assert cfg == M.default_phi3_config()
    # the probe table is the stream_llm heads of the original best pattern
    assert [list(t) for t in M.PHI3_PROBE_HEADS] == golden["best_pattern"]["stream_scores"]
    # the benchmark's all-sparse mix stays available by path
    mix = json.load(open(M.NAMED_CONFIGS["phi3_stream_block_50_50"]))
    kinds = [rec[0] for layer in mix for rec in layer.values()]
    assert kinds.count("stream_llm") == 512 and kinds.count("block_sparse") == 512
    assert mix == P.headline_config(seed=0)


def test_mixed_config_counts_and_seed():
    mix = [(0.3, P.record("stream_llm", 128, 4096)), (0.6, P.record("block_sparse", 100)),
           (0.1, P.record("dense"))]
    a, b = P.mixed_config(mix, seed=3), P.mixed_config(mix, seed=3)
    assert a == b
    kinds = [rec[0] for layer in a for rec in layer.values()]
    assert (kinds.count("stream_llm"), kinds.count("block_sparse"), kinds.count("dense")) == (307, 614, 103)


def test_load_layer_patterns(tmp_path):
    path = tmp_path / "p.json"
    P.write(str(path), P.uniform_config("block_sparse", 8, n_layers=2, n_heads=3))
    pats = MF.load_layer_patterns(str(path), 1)
    assert pats == {0: ["block_sparse", 8, 0, 1.0], 1: ["block_sparse", 8, 0, 1.0],
                    2: ["block_sparse", 8, 0, 1.0]}
    assert MF.load_layer_patterns(str(path), 5) == {}
    assert MF.load_layer_patterns(str(tmp_path / "missing.json"), 0) == {}


def test_build_layer_plan_semantics():
    pats = {0: ["stream_llm", 100, 800, 0.9], 1: ["block_sparse", 1000, 0, 1.0],
            2: ["dense", 0, 0, 1.0], 3: ["block_sparse", 0, 0, 1.0]}
    plan = MF.build_layer_plan(pats, 4, 96, 4096)
    s_sp, s_de = 128 ** -0.5, 1.0 / math.sqrt(96)  # dense: 1/sqrt(D) as attention.py:210-211
    assert plan.heads[0] == (_abi.MSA_KIND_STREAM, 100, 800, -1, s_sp)
    assert plan.heads[1] == (_abi.MSA_KIND_BLOCK, 64, 0, 0, s_sp)   # clamped to n_blocks
    assert plan.heads[2] == (_abi.MSA_KIND_DENSE, 0, 0, -1, s_de)
    assert plan.heads[3] == (_abi.MSA_KIND_BLOCK, 1, 0, 1, s_sp)    # clamped to >= 1
    assert plan.block_heads == (1, 3) and plan.block_topk == (64, 1) and plan.topk_max == 64
    assert not plan.all_dense and plan.vs_heads == ()
    # head 1 missing -> the default record ("vertical_and_slash", 1000, 6096, 1),
    # counts clamped to min(S, max(v, 30)) and min(S, max(s, 50)) (:146-147)
    vs = MF.build_layer_plan({0: pats[0]}, 2, 96, 4096)
    assert vs.heads[1] == (_abi.MSA_KIND_VS, 1000, 4096, 0, s_sp)
    assert vs.vs_heads == (1,) and vs.vs_counts == ((1000, 4096),)
    small = MF.build_layer_plan({0: ["vertical_and_slash", 10, 20, 1]}, 1, 96, 40)
    assert small.heads[0] == (_abi.MSA_KIND_VS, 30, 40, 0, s_sp)
    with pytest.raises(ValueError):
        MF.build_layer_plan({0: ["a_shape", 1, 2, 3]}, 1, 96, 4096)


# ---------------------------------------------------------------------------
# HF patch plumbing on a tiny Phi-3 (CPU, test double for the launch)
# ---------------------------------------------------------------------------
def _oracle_launch(q, k, v, plan, out):
    """CPU stand-in for run_layer_attention: the oracle per head kind."""
    qn = q.detach().float().numpy()
    kn = k.detach().float().numpy()
    vn = v.detach().float().numpy()
    H, Hkv = qn.shape[1], kn.shape[1]
    rep = H // Hkv
    kn, vn = np.repeat(kn, rep, 1), np.repeat(vn, rep, 1)
    res = np.zeros(qn.shape)
    for h, (kind, p1, p2, slot, scale) in enumerate(plan.heads):
        sl = slice(h, h + 1)
        if kind == _abi.MSA_KIND_STREAM:
            res[:, sl] = O.streaming_attention(qn[:, sl], kn[:, sl], vn[:, sl], p1, p2, scale=scale)
        elif kind == _abi.MSA_KIND_BLOCK:
            idx, _ = O.select_block_sparse_topk_indices(qn[:, sl], kn[:, sl], p1, "fp32", scale)
            res[:, sl] = O.block_sparse_from_indices(qn[:, sl], kn[:, sl], vn[:, sl], idx, scale=scale)
        elif kind == _abi.MSA_KIND_VS:
            vi, si = O.vs_estimate(qn[:, sl], kn[:, sl], p1, p2, "fp32")
            res[:, sl] = O.vertical_slash_from_indices(qn[:, sl], kn[:, sl], vn[:, sl], vi, si,
                                                       scale=scale)
        else:
            res[:, sl] = O.dense_causal(qn[:, sl], kn[:, sl], vn[:, sl], scale=scale)
    out.copy_(torch.from_numpy(res).to(out.dtype))
    return out


def _tiny_phi3(n_heads=2, n_kv=2, layers=2, seed=0):
    from transformers import Phi3Config, Phi3ForCausalLM

    torch.manual_seed(seed)
    cfg = Phi3Config(hidden_size=96 * n_heads, intermediate_size=256, num_hidden_layers=layers,
                     num_attention_heads=n_heads, num_key_value_heads=n_kv, vocab_size=128,
                     max_position_embeddings=4096, pad_token_id=0, bos_token_id=1,
                     eos_token_id=2)
    return Phi3ForCausalLM(cfg).eval()


def _oracle_decode(q, k, v, out, scale):
    """CPU stand-in for run_decode_attention: the last query row sees every key."""
    qn = q.detach().float().numpy()
    kn = k.detach().float().numpy()
    vn = v.detach().float().numpy()
    rep = qn.shape[1] // kn.shape[1]
    kn, vn = np.repeat(kn, rep, 1), np.repeat(vn, rep, 1)
    res = O.dense_causal(qn, kn, vn, scale=scale)
    out.copy_(torch.from_numpy(res).to(out.dtype))
    return out


@pytest.fixture
def cpu_launch(monkeypatch):
    monkeypatch.setattr(MF, "run_layer_attention", _oracle_launch)
    monkeypatch.setattr(MF, "run_decode_attention", _oracle_decode)


@pytest.mark.parametrize("n_kv", [2, 1])
def test_patched_dense_matches_hf(tmp_path, cpu_launch, n_kv):
    model = _tiny_phi3(n_kv=n_kv)
    ids = torch.randint(3, 128, (1, 150), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        ref = model(ids).logits
    path = tmp_path / "dense.json"
    P.write(str(path), P.uniform_config("dense", n_layers=2, n_heads=2))
    patched = MInference(attn_type="minference", config_path=str(path))(model)
    assert patched.config._attn_implementation == "minference"
    assert patched.config.minference_attn_type == "minference"
    with torch.no_grad():
        got = patched(ids).logits
    assert torch.allclose(got, ref, atol=2e-4, rtol=1e-3), (got - ref).abs().max()


def test_patched_decode_with_cache_matches_hf(tmp_path, cpu_launch):
    model = _tiny_phi3()
    ids = torch.randint(3, 128, (1, 40), generator=torch.Generator().manual_seed(2))
    with torch.no_grad():
        ref = model.generate(ids, max_new_tokens=4, do_sample=False, use_cache=True)
    path = tmp_path / "dense.json"
    P.write(str(path), P.uniform_config("dense", n_layers=2, n_heads=2))
    patched = MInference(attn_type="minference", config_path=str(path))(model)
    with torch.no_grad():
        got = patched.generate(ids, max_new_tokens=4, do_sample=False, use_cache=True)
    assert torch.equal(got, ref)


def test_patched_sparse_layer_uses_plan(tmp_path, cpu_launch, monkeypatch):
    """stream_llm / block_sparse heads reach the launch with the reference's
    parameters and scale, and starting_layer keeps early layers dense."""
    seen = []

    def spy(q, k, v, plan, out):
        seen.append(plan)
        return _oracle_launch(q, k, v, plan, out)

    monkeypatch.setattr(MF, "run_layer_attention", spy)
    model = _tiny_phi3()
    path = tmp_path / "mix.json"
    cfg = [{"0": ["stream_llm", 16, 64, 1.0], "1": ["block_sparse", 2, 0, 1.0]}] * 2
    P.write(str(path), cfg)
    patched = patch_hf(model, "minference", {"config_path": str(path), "starting_layer": 1})
    ids = torch.randint(3, 128, (1, 200), generator=torch.Generator().manual_seed(3))
    with torch.no_grad():
        patched(ids)
    assert seen[0].all_dense and seen[0].heads[0][4] == 1.0 / math.sqrt(96)  # layer 0 < starting_layer
    assert seen[1].heads[0] == (_abi.MSA_KIND_STREAM, 16, 64, -1, 128 ** -0.5)
    assert seen[1].heads[1] == (_abi.MSA_KIND_BLOCK, 2, 0, 0, 128 ** -0.5)


def _mask_spy(model):
    """Wraps every attention module's forward to record the attention_mask
    it receives."""
    seen = []
    for layer in model.model.layers:
        attn = layer.self_attn
        inner = attn.forward

        def spy(*a, _inner=inner, **kw):
            seen.append(kw.get("attention_mask", a[2] if len(a) > 2 else None))
            return _inner(*a, **kw)

        attn.forward = spy
    return seen


def test_patched_layers_receive_no_mask(tmp_path, cpu_launch):
    """The 4D-mask skip (reference minference/patch.py:39-87): under the
    "minference" implementation HF builds no [B, 1, S, S] mask and every
    patched layer gets attention_mask=None (a 128K eager mask is 34 GB).  The
    unpatched eager model on the same ids does get a 4D mask, so the spy
    sees what it claims to."""
    ids = torch.randint(3, 128, (1, 96), generator=torch.Generator().manual_seed(5))
    eager = _tiny_phi3()
    eager.set_attn_implementation("eager")
    seen_eager = _mask_spy(eager)
    with torch.no_grad():
        eager(ids)
    assert len(seen_eager) == 2
    assert all(isinstance(m, torch.Tensor) and m.dim() == 4 for m in seen_eager)

    path = tmp_path / "dense.json"
    P.write(str(path), P.uniform_config("dense", n_layers=2, n_heads=2))
    patched = MInference(attn_type="minference", config_path=str(path))(_tiny_phi3())
    seen = _mask_spy(patched)
    with torch.no_grad():
        patched(ids, attention_mask=torch.ones_like(ids))
        patched(ids)
    assert len(seen) == 4 and all(m is None for m in seen)


def test_more_heads_than_one_launch_raises(monkeypatch):
    """A layer with more than MSA_MAX_HEADS query heads is refused with a
    clear error before any launch (no recursion through batch slices)."""
    monkeypatch.setattr(_abi, "require_device", lambda *t: None)
    H = _abi.MSA_MAX_HEADS + 8
    plan = MF.build_layer_plan({}, H, 64, 64)  # every head defaults to vertical_and_slash
    q = torch.zeros(2, H, 64, 64, dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError, match="heads"):
        MF.run_layer_attention(q, q, q, plan, torch.empty_like(q))
    dense = MF.dense_plan(H, 64)
    with pytest.raises(NotImplementedError, match="heads"):
        MF.run_layer_attention(q, q, q, dense, torch.empty_like(q))


def test_hf_attn_type_leaves_model_unpatched():
    model = _tiny_phi3()
    fwd = model.model.layers[0].self_attn.forward
    assert MInference(attn_type="hf")(model) is model
    assert model.model.layers[0].self_attn.forward == fwd


def test_missing_heads_run_vertical_and_slash(tmp_path, monkeypatch):
    """A head absent from the JSON takes the reference default
    ("vertical_and_slash", 1000, 6096, 1) (minference_forward.py:229-231)."""
    seen = []

    def spy(q, k, v, plan, out):
        seen.append(plan)
        return _oracle_launch(q, k, v, plan, out)

    monkeypatch.setattr(MF, "run_layer_attention", spy)
    model = _tiny_phi3()
    path = tmp_path / "partial.json"
    P.write(str(path), [{"0": ["stream_llm", 16, 64, 1.0]}] * 2)
    patched = patch_hf(model, "minference", {"config_path": str(path)})
    ids = torch.randint(3, 128, (1, 150), generator=torch.Generator().manual_seed(4))
    with torch.no_grad():
        logits = patched(ids).logits
    assert torch.isfinite(logits).all()
    assert seen[0].heads[1] == (_abi.MSA_KIND_VS, 150, 150, 0, 128 ** -0.5)
    assert seen[0].vs_heads == (1,)


def test_vertical_and_slash_needs_full_prefill():
    """vertical_slash_kernel_npu.py:551-556: S_q != S_k is an AssertionError."""
    plan = MF.build_layer_plan({0: ["vertical_and_slash", 100, 200, 1]}, 1, 96, 300)
    q = torch.zeros(1, 1, 100, 96, dtype=torch.bfloat16)
    k = torch.zeros(1, 1, 300, 96, dtype=torch.bfloat16)
    with pytest.raises(AssertionError):
        MF._vs_lists(q, k, plan)


def test_patch_time_pattern_check_warns(tmp_path):
    """The pattern file is validated against the model once at patch time;
    problems warn (the reference only fails in the forward that reaches a bad
    record) and a clean file is silent."""
    import warnings

    bad = tmp_path / "bad.json"
    P.write(str(bad), [{"0": ["stream_llm", 16, 64, 1.0], "5": ["dense", 0, 0, 1.0]}] * 3)
    with pytest.warns(UserWarning, match=r"head 5 >= 2 heads.*|3 layers, the model has 2"):
        patch_hf(_tiny_phi3(), "minference", {"config_path": str(bad)})
    good = tmp_path / "good.json"
    P.write(str(good), P.uniform_config("block_sparse", 4, n_layers=2, n_heads=2))
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        patch_hf(_tiny_phi3(), "minference", {"config_path": str(good)})


def test_is_search_runs_layers_dense(tmp_path, monkeypatch):
    """is_search=True warns and runs every layer dense (reference
    minference_forward.py:374-382, :392-396), whatever the pattern file says."""
    seen = []

    def spy(q, k, v, plan, out):
        seen.append(plan)
        return _oracle_launch(q, k, v, plan, out)

    monkeypatch.setattr(MF, "run_layer_attention", spy)
    path = tmp_path / "mix.json"
    P.write(str(path), [{"0": ["stream_llm", 16, 64, 1.0], "1": ["block_sparse", 2, 0, 1.0]}] * 2)
    patched = MInference(attn_type="minference", config_path=str(path), is_search=True)(_tiny_phi3())
    ids = torch.randint(3, 128, (1, 100), generator=torch.Generator().manual_seed(5))
    with pytest.warns(UserWarning, match="is_search"), torch.no_grad():
        patched(ids)
    assert len(seen) == 2 and all(p.all_dense for p in seen)
    assert seen[0].heads[0][4] == 1.0 / math.sqrt(96)

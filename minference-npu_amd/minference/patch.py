"""HF transformers patch: drop-in for MInference-NPU/minference/patch.py:90-159.

``minference_patch`` rebinds ``forward`` of every attention module of the
model's attention class (as the reference does, :101-127) and, for the
installed transformers (5.x), registers a ``"minference"`` attention
implementation whose mask function returns None so the model never builds the
[B, 1, S, S] causal mask (the reference's 4D-mask skip helper, :39-87, has no
effect on transformers 5.x).  Unpatched attention modules that still reach the
registered attention function run the HIP dense kernel.
"""

from __future__ import annotations

import json
import os
import warnings
from typing import Any

import torch

from .modules.minference_forward import init_minference_parameters, minference_forward

__all__ = [
    "minference_patch",
    "patch_hf",
    "register_attention_implementation",
    "minference_patch_kv_cache_cpu",
    "minference_patch_with_kvcompress",
    "minference_patch_vllm",
    "new_patch",
]

ATTN_IMPL = "minference"
_REGISTERED = False


def _no_mask(*args, attention_mask=None, **kwargs):
    """Mask function of the "minference" implementation: the patched forward
    applies the causal/sparse masks inside the kernels and ignores HF's mask,
    as the reference's patched forward does."""
    if isinstance(attention_mask, torch.Tensor) and attention_mask.dim() == 2:
        if bool((attention_mask == 0).any().item()):
            warnings.warn("padding in attention_mask is ignored by the minference attention",
                          stacklevel=2)
    return None


def _dense_attention_interface(module, query, key, value, attention_mask, scaling=None,
                               dropout=0.0, **kwargs):
    """AttentionInterface entry: causal dense attention on the HIP kernel.
    Returns ([B, S, H, D], None) like HF's sdpa/eager functions."""
    from .modules.minference_forward import dense_plan, run_layer_attention

    bsz, n_heads, q_len, hd = query.shape
    out_bshd = torch.empty((bsz, q_len, n_heads, hd), dtype=query.dtype, device=query.device)
    run_layer_attention(query, key, value, dense_plan(n_heads, hd, scaling), out_bshd.transpose(1, 2))
    return out_bshd, None


def register_attention_implementation() -> str:
    """Register the "minference" attention + mask implementations with HF."""
    global _REGISTERED
    if not _REGISTERED:
        from transformers.masking_utils import AttentionMaskInterface
        from transformers.modeling_utils import AttentionInterface

        AttentionInterface.register(ATTN_IMPL, _dense_attention_interface)
        AttentionMaskInterface.register(ATTN_IMPL, _no_mask)
        _REGISTERED = True
    return ATTN_IMPL


def _check_pattern_file(config: Any, model_config: Any) -> None:
    """Validate the pattern file against the model's layer and head counts
    once, at patch time.  Problems are warnings, not errors: the reference
    dispatcher reads the file lazily per layer (minference_forward.py:187-198)
    and fails, if at all, only in the forward that reaches the bad record."""
    path = getattr(config, "config_path", "")
    if getattr(config, "attn_type", "") != "minference" or not path or not os.path.exists(path):
        return
    from .configs.patterns import PatternConfigError, validate_config

    try:
        with open(path) as f:
            cfg = json.load(f)
        validate_config(cfg, getattr(model_config, "num_hidden_layers", None),
                        getattr(model_config, "num_attention_heads", None), where=path)
    except (ValueError, PatternConfigError) as e:
        warnings.warn(f"pattern file check failed: {e}", stacklevel=3)


def minference_patch(model: torch.nn.Module, config: Any) -> torch.nn.Module:
    """Bind the MI355X minference forward onto ``model.model.layers[*].self_attn``.

    Args:
        model:  HF causal LM (Phi-3 family; Llama-style ``model.model.layers``)
        config: MInferenceConfig (attn_type / starting_layer / config_path are read)
    """
    try:
        attention_module = model.model.layers[0].self_attn
    except AttributeError as e:
        raise RuntimeError(
            "model.model.layers[0].self_attn not found; only Llama/Phi-style models are supported"
        ) from e

    AttentionClass = attention_module.__class__
    forward_closure = minference_forward()
    _check_pattern_file(config, model.config)

    model.config.starting_layer = config.starting_layer
    model.config.config_path = config.config_path
    model.config.minference_attn_type = config.attn_type
    model.config.is_search = getattr(config, "is_search", False)

    impl = register_attention_implementation()
    try:
        model.set_attn_implementation(impl)
    except Exception:  # noqa: BLE001 - older transformers: set the field directly
        model.config._attn_implementation = impl

    def update_module(m: torch.nn.Module) -> None:
        if isinstance(m, AttentionClass):
            m._minference_initialized = False
            m.init_minference_parameters = init_minference_parameters.__get__(m, AttentionClass)
            m.forward = forward_closure.__get__(m, AttentionClass)

    model.apply(update_module)
    print(
        f"[MInference-MI355X] Patched {AttentionClass.__name__}.forward "
        f"(starting_layer={config.starting_layer}, attn_type={config.attn_type})"
    )
    return model


def patch_hf(
    model: torch.nn.Module,
    attn_type: str = "minference",
    attn_kwargs: dict | None = None,
    **kwargs: Any,
) -> torch.nn.Module:
    """Compatibility entry matching the reference ``patch_hf`` (:135-159)."""
    attn_kwargs = dict(attn_kwargs or {})
    attn_kwargs.update(kwargs)
    if attn_type not in ("minference", "dense"):
        raise NotImplementedError(
            f"patch_hf attn_type={attn_type!r} is not supported; use 'minference' or 'dense'"
        )
    from .minference_configuration import MInferenceConfig

    config = MInferenceConfig(
        attn_type=attn_type,
        attn_kwargs=attn_kwargs,
        starting_layer=attn_kwargs.get("starting_layer", -1),
        config_path=attn_kwargs.get("config_path"),
    )
    return minference_patch(model, config)


def minference_patch_kv_cache_cpu(model):
    raise NotImplementedError("KV cache CPU offload is not part of this build")


def minference_patch_with_kvcompress(model, config):
    raise NotImplementedError("KV compression is not part of this build")


def minference_patch_vllm(*args, **kwargs):
    raise NotImplementedError("vLLM integration is not part of this build")


def new_patch(model, config):
    raise NotImplementedError(
        f"new_patch (attn_type={config.attn_type!r}, kv_type={config.kv_type!r}) is not part of this build"
    )

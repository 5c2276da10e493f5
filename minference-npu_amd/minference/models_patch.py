"""Top-level patch entry: drop-in for MInference-NPU/minference/models_patch.py:26-94."""

from __future__ import annotations

import json
import os

from .minference_configuration import MInferenceConfig

os.environ.setdefault("TOKENIZERS_PARALLELISM", "false")

_SUPPORTED_ATTN = ("minference", "dense", "hf")
_SUPPORTED_KV = ("dense",)


class MInference:
    """``model = MInference(attn_type="minference", model_name=...)(model)``.

    attn_type "hf" leaves the model untouched, "dense" runs every head on the
    dense HIP kernel, "minference" dispatches each head by its pattern.
    """

    def __init__(
        self,
        attn_type: str = "minference",
        model_name: str | None = None,
        config_path: str | None = None,
        starting_layer: int = -1,
        kv_type: str = "dense",
        is_search: bool = False,
        attn_kwargs: dict | None = None,
        **kwargs,
    ):
        if attn_type not in _SUPPORTED_ATTN:
            raise ValueError(f"attn_type={attn_type!r} is not supported; use one of {_SUPPORTED_ATTN}")
        if kv_type not in _SUPPORTED_KV:
            raise ValueError(f"kv_type={kv_type!r} is not supported; use one of {_SUPPORTED_KV}")
        self.config = MInferenceConfig(
            attn_type=attn_type,
            model_name=model_name,
            config_path=config_path,
            starting_layer=starting_layer,
            kv_cache_cpu=False,
            kv_type=kv_type,
            is_search=is_search,
            attn_kwargs=attn_kwargs or {},
            **kwargs,
        )

    def __call__(self, model):
        return self.patch_model(model)

    def patch_model(self, model):
        if self.config.attn_type == "hf":
            return model
        if self.config.attn_type == "minference" and not self.config.is_search:
            if not self.config.config_path:
                raise ValueError(
                    "attn_type='minference' needs model_name (MODEL2PATH) or config_path"
                )
            with open(self.config.config_path, "r") as f:
                self.config.attn_kwargs.setdefault("best_pattern", json.load(f))
        from .patch import minference_patch

        return minference_patch(model, self.config)

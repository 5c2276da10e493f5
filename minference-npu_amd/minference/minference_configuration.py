"""Configuration object of the drop-in API.

Interface (names, keyword arguments and their defaults, the attribute set
and the error class for an unsupported choice) follows
MInference-NPU/minference/minference_configuration.py:7-75, so user code that
builds an ``MInferenceConfig`` by keyword runs unchanged.  The behaviour is
this build's own: a small table normalises legacy spellings, the pattern
file is resolved once at construction, and every rejected choice names the
accepted ones.
"""

from __future__ import annotations

from typing import Any, Dict, Optional, Tuple

from .configs.model2path import MODEL2PATH

# Legacy spellings accepted at construction and what they mean here.
_ATTN_ALIASES = {"minference_with_dense": "dense"}
_KV_ALIASES = {"": "dense"}


class MInferenceConfig:
    """What ``MInference`` / ``minference_patch`` need to patch a model.

    attn_type "minference" runs the per-head sparse patterns of a pattern
    file (``config_path``, or the file registered for ``model_name``); "hf"
    and "dense" leave attention dense and need no file (``config_path`` is
    then "").  Only the dense KV cache exists on this path."""

    MINFERENCE_ATTENTION_TYPES = ["minference"]
    OTHER_ATTENTION_TYPES = ["hf", "dense"]
    KV_TYPES = ["dense"]

    def __init__(
        self,
        attn_type: str = "minference",
        model_name: str = None,
        config_path: str = None,
        starting_layer: int = -1,
        kv_cache_cpu: bool = False,
        kv_cache_cpu_device: str = "cpu",
        kv_type: str = "dense",
        is_search: bool = False,
        attn_kwargs: Optional[Dict[str, Any]] = None,
        **kwargs,
    ):
        self.attn_type, self.kv_type = self.update_config_type(attn_type, kv_type)
        _require(self.attn_type, self.get_available_attn_types(), "attn_type")
        _require(self.kv_type, self.get_available_kv_types(), "kv_type")
        self.model_name = model_name
        self.config_path = self.update_config_path(config_path, model_name)
        self.starting_layer = starting_layer
        self.is_search = is_search
        self.kv_cache_cpu = kv_cache_cpu
        self.kv_cache_cpu_device = kv_cache_cpu_device
        # what the patched layers read (init_minference_parameters); caller
        # entries override the three derived ones
        derived = {"is_search": is_search, "starting_layer": starting_layer,
                   "config_path": self.config_path}
        self.attn_kwargs = {**derived, **dict(attn_kwargs or {})}

    def update_config_path(self, config_path: str = None, model_name: str = None) -> str:
        """Pattern file of this configuration: none for the dense types, an
        explicit path as given, else the file registered for the model."""
        if self.attn_type not in self.MINFERENCE_ATTENTION_TYPES:
            return ""
        if config_path is not None:
            return config_path
        if model_name not in MODEL2PATH:
            known = ", ".join(sorted(MODEL2PATH)) or "none"
            raise AssertionError(f"no pattern file is registered for model {model_name!r} "
                                 f"(registered: {known}); pass config_path instead")
        return MODEL2PATH[model_name]

    def get(self, attr: str, default=None):
        return getattr(self, attr, default)

    @staticmethod
    def update_config_type(attn_type: str, kv_type: str) -> Tuple[str, str]:
        """Maps legacy spellings to the names this build dispatches on."""
        return _ATTN_ALIASES.get(attn_type, attn_type), _KV_ALIASES.get(kv_type, kv_type)

    @classmethod
    def get_available_attn_types(cls):
        return [*cls.MINFERENCE_ATTENTION_TYPES, *cls.OTHER_ATTENTION_TYPES]

    @classmethod
    def get_available_kv_types(cls):
        return list(cls.KV_TYPES)


def _require(value: str, allowed, what: str) -> None:
    # AssertionError is the reference's error class for these choices.
    if value not in allowed:
        raise AssertionError(f"{what} {value!r} is not supported; choose one of {allowed}")

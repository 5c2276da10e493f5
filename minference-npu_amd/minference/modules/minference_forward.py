"""Patched attention forward: per-head pattern dispatch in one launch per layer.

Drop-in for MInference-NPU/minference/modules/minference_forward.py:
  init_minference_parameters  :175-213  (per-layer pattern load)
  minference_forward          :258-502  (the patched forward)
The reference groups heads by (type, params) and runs gather -> op -> scatter
per group (:398-487).  Here the layer's heads become a descriptor table
(LayerPlan); the block_sparse heads share one estimator launch, the
vertical_and_slash heads another, and one library call runs the attention of
every head (vertical_and_slash heads in their own kernel launch), writing the
output in [B, S, H, D] order, so the o_proj input needs no transpose copy.

Written against the installed transformers (5.x): the attention module gets
``position_embeddings`` from the model and returns a 2-tuple.
"""

from __future__ import annotations

import json
import math
import os
import warnings
from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence, Tuple

import torch

from .. import _abi
from ..ops.common import VS_HEAD_DIMS, dense_scale, require_kernel_head_dim, sparse_scale
from ..ops.rope import apply_rotary_pos_emb as apply_rotary_pos_emb_gpu, rope_supported
from ..ops.vertical_slash_kernel import vs_sizes

__all__ = [
    "DEFAULT_PATTERN",
    "LayerPlan",
    "build_layer_plan",
    "init_minference_parameters",
    "load_layer_patterns",
    "minference_forward",
    "run_layer_attention",
]

# A head missing from the JSON gets this record (reference :229-231, :405-407).
DEFAULT_PATTERN = ("vertical_and_slash", 1000, 6096, 1)

_KIND = {
    "dense": _abi.MSA_KIND_DENSE,
    "stream_llm": _abi.MSA_KIND_STREAM,
    "block_sparse": _abi.MSA_KIND_BLOCK,
}


def load_layer_patterns(config_path: str, layer_idx: int) -> Dict[int, list]:
    """``{head: [type, p1, p2, score]}`` of one layer from the pattern JSON
    (a list with one ``{"head": record}`` dict per layer; reference :187-198).
    A missing file or layer yields ``{}``."""
    if not config_path or not os.path.exists(config_path):
        return {}
    with open(config_path) as f:
        all_patterns = json.load(f)
    if layer_idx < len(all_patterns):
        return {int(h): rec for h, rec in all_patterns[layer_idx].items()}
    return {}


@dataclass(frozen=True)
class LayerPlan:
    """Head descriptor table of one layer for a given K length.

    heads[h] = (kind, p1, p2, slot, scale) as passed to msa_layer_attention;
    block_heads[s] / block_topk[s] = head and clamped top-k of estimator slot s;
    vs_heads[s] / vs_counts[s] = head and clamped (vertical, slash) counts of
    vertical_and_slash slot s.
    """

    heads: Tuple[tuple, ...]
    block_heads: Tuple[int, ...]
    block_topk: Tuple[int, ...]
    topk_max: int
    all_dense: bool
    vs_heads: Tuple[int, ...] = ()
    vs_counts: Tuple[Tuple[int, int], ...] = ()


def build_layer_plan(patterns: Dict[int, Sequence], n_heads: int, head_dim: int,
                     s_k: int, layer_idx: Optional[int] = None) -> LayerPlan:
    """Per-head semantics of the reference dispatcher (:404-419, :228-250):

    * ``stream_llm``  : p1 = n_init, p2 = n_local, scale (padded D)**-0.5
    * ``block_sparse``: p1 = top-k key blocks, clamped to [1, n_k_blocks],
                        scale (padded D)**-0.5 (selector and attention)
    * ``dense``       : causal dense, scale 1/sqrt(D)
    * ``vertical_and_slash`` (also the default for a missing head, :229-231):
                        p1 = vertical count, p2 = slash count, clamped to
                        min(S, max(p1, 30)) / min(S, max(p2, 50)) (:146-147);
                        estimator scale 1/sqrt(D), attention scale (padded
                        D)**-0.5 (vertical_slash_kernel_npu.py:581-587)
    Unknown types raise ValueError as in the reference (:416-419).
    """
    n_kb = max(1, math.ceil(s_k / _abi.MSA_BLOCK))
    s_sparse = sparse_scale(head_dim)
    s_dense = dense_scale(head_dim)
    heads: List[tuple] = []
    block_heads: List[int] = []
    block_topk: List[int] = []
    vs_heads: List[int] = []
    vs_counts: List[Tuple[int, int]] = []
    for h in range(n_heads):
        rec = patterns.get(h, DEFAULT_PATTERN)
        ty, p1, p2 = rec[0], rec[1], rec[2]
        if ty == "stream_llm":
            heads.append((_abi.MSA_KIND_STREAM, int(p1), int(p2), -1, s_sparse))
        elif ty == "block_sparse":
            k = min(max(1, int(p1)), n_kb)
            heads.append((_abi.MSA_KIND_BLOCK, k, 0, len(block_heads), s_sparse))
            block_heads.append(h)
            block_topk.append(k)
        elif ty == "dense":
            heads.append((_abi.MSA_KIND_DENSE, 0, 0, -1, s_dense))
        elif ty == "vertical_and_slash":
            nv, ns = vs_sizes(s_k, p1, p2)
            heads.append((_abi.MSA_KIND_VS, nv, ns, len(vs_heads), s_sparse))
            vs_heads.append(h)
            vs_counts.append((nv, ns))
        else:
            raise ValueError(f"unknown best_pattern type {ty!r} (layer={layer_idx} head={h})")
    return LayerPlan(
        heads=tuple(heads),
        block_heads=tuple(block_heads),
        block_topk=tuple(block_topk),
        topk_max=max(block_topk) if block_topk else 0,
        all_dense=all(hd[0] == _abi.MSA_KIND_DENSE for hd in heads),
        vs_heads=tuple(vs_heads),
        vs_counts=tuple(vs_counts),
    )


def dense_plan(n_heads: int, head_dim: int, scale: Optional[float] = None) -> LayerPlan:
    s = dense_scale(head_dim) if scale is None else float(scale)
    return LayerPlan(
        heads=tuple((_abi.MSA_KIND_DENSE, 0, 0, -1, s) for _ in range(n_heads)),
        block_heads=(), block_topk=(), topk_max=0, all_dense=True,
    )


def _vs_lists(q: torch.Tensor, k: torch.Tensor, plan: LayerPlan):
    """Estimator launch for the vertical_and_slash heads: (v_idx, v_cnt, s_idx,
    s_cnt) for msa_layer_attention_ex."""
    assert q.shape[2] == k.shape[2], (
        "vertical_and_slash heads need S_q == S_k (full prefill); got "
        f"S_q={q.shape[2]}, S_k={k.shape[2]}"
    )
    if q.shape[2] > _abi.MSA_VS_MAX_SEQ:
        raise NotImplementedError(
            f"vertical_and_slash supports S <= {_abi.MSA_VS_MAX_SEQ} on MI355X, got {q.shape[2]}"
        )
    B = q.shape[0]
    n = len(plan.vs_heads)
    nv = max(c[0] for c in plan.vs_counts)
    ns = max(c[1] for c in plan.vs_counts)
    dev = q.device
    v_idx = torch.empty((B, n, nv), dtype=torch.int32, device=dev)
    s_idx = torch.empty((B, n, ns), dtype=torch.int32, device=dev)
    v_cnt = torch.empty((B, n), dtype=torch.int32, device=dev)
    s_cnt = torch.empty((B, n), dtype=torch.int32, device=dev)
    _abi.vs_estimate(q, k, plan.vs_heads, [c[0] for c in plan.vs_counts],
                     [c[1] for c in plan.vs_counts], v_idx, v_cnt, s_idx, s_cnt)
    return v_idx, v_cnt, s_idx, s_cnt


def run_layer_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, plan: LayerPlan,
                        out: torch.Tensor) -> torch.Tensor:
    """Estimator launches (block_sparse and vertical_and_slash heads) + one
    attention call for all heads (launch_block_layer's schedule for a layer
    with block_sparse heads and no vertical_and_slash heads).

    q [B, H, S_q, D]; k/v [B, H_kv, S_k, D] (H % H_kv == 0, no repeat_kv copy);
    out any [B, H, S_q, D] view with D contiguous (bf16/fp16 or fp32).
    """
    _abi.require_device(q, k, v)
    require_kernel_head_dim(q.shape[-1], "the patched attention forward")
    if plan.vs_heads:
        require_kernel_head_dim(q.shape[-1], "vertical_and_slash heads", VS_HEAD_DIMS)
    B, H, S_q, _ = q.shape
    if H > _abi.MSA_MAX_HEADS:
        raise NotImplementedError(
            f"one attention launch takes at most {_abi.MSA_MAX_HEADS} query heads, got {H}")
    if plan.vs_heads and B * H > _abi.MSA_MAX_HEADS:
        # vertical_and_slash layers run in batch slices of at most MSA_MAX_HEADS heads
        step = max(1, _abi.MSA_MAX_HEADS // H)
        for b0 in range(0, B, step):
            b1 = min(B, b0 + step)
            run_layer_attention(q[b0:b1], k[b0:b1], v[b0:b1], plan, out[b0:b1])
        return out
    n_slots = len(plan.block_heads)
    if not n_slots and not plan.vs_heads:
        _abi.layer_attention(q, k, v, out, plan.heads)
        return out
    ws = _abi.workspace(_abi.attention_workspace_bytes(k.shape[0], k.shape[1], k.shape[2],
                                                       k.shape[3]), q.device)
    idx = cnt = None
    if n_slots:
        n_qb = math.ceil(S_q / _abi.MSA_BLOCK)
        idx = torch.empty((B, n_slots, n_qb, plan.topk_max), dtype=torch.int32, device=q.device)
        cnt = torch.empty((B, n_slots, n_qb), dtype=torch.int32, device=q.device)
    if not plan.vs_heads:
        est_ws = _abi.workspace(_abi.estimate_workspace_bytes(B, n_slots, S_q, k.shape[2],
                                                              q.shape[3]), q.device)
        launch_block_layer(q, k, v, plan, out, idx, cnt, ws, est_ws)
        return out
    # vertical_and_slash heads: K/V staging on the side stream under the
    # estimators, then one attention call for all heads
    main = torch.cuda.current_stream(q.device)
    side = _side_stream(q.device)
    side.wait_stream(main)
    with torch.cuda.stream(side):
        _abi.stage_kv(k, v, ws)
    if n_slots:
        _abi.block_estimate(q, k, plan.block_heads, plan.block_topk, plan.topk_max,
                            sparse_scale(q.shape[-1]), idx, cnt)
    vs = _vs_lists(q, k, plan)
    main.wait_stream(side)
    _abi.layer_attention(q, k, v, out, plan.heads, idx=idx, cnt=cnt, idx_slots=n_slots,
                         topk_max=plan.topk_max, ws=ws, staged=True, vs=vs)
    return out


def launch_block_layer(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, plan: LayerPlan,
                       out: torch.Tensor, idx: torch.Tensor, cnt: torch.Tensor,
                       ws: torch.Tensor, est_ws: torch.Tensor, flags: int = 0,
                       mark=None) -> None:
    """Launches of a layer with block_sparse heads and no vertical_and_slash
    heads, in order on the current stream:

      1. K/V staging and the block estimator's pooling pass, one launch
         (msa_stage_kv_pool; then the small V-range pass);
      2. the block selection: scores and top-k (msa_block_estimate_ex,
         MSA_ESTIMATE_SELECT_ONLY);
      3. one attention launch of all heads.

    One stream and no events between the launches: each launch starts as the
    previous one drains (cross-stream waits cost 10-20 us each here).  Every
    head of the layer is in the one attention grid, whatever the pattern mix.
    ``est_ws`` is the estimator workspace both estimator passes share.
    ``mark(name, stream)``, when given, is called at the phase boundaries
    ("start", "stage0", "stage1", "est0", "est1", "attn0", "attn0_end"; the
    benchmark records events there)."""
    mark = mark or (lambda name, stream: None)
    main = torch.cuda.current_stream(q.device)
    mark("start", main)
    mark("stage0", main)
    _abi.stage_kv_pool(q, k, v, plan.block_heads, est_ws, ws)
    mark("stage1", main)
    mark("est0", main)
    _abi.block_estimate(q, k, plan.block_heads, plan.block_topk, plan.topk_max,
                        sparse_scale(q.shape[-1]), idx, cnt, est_ws,
                        flags=flags | _abi.MSA_ESTIMATE_SELECT_ONLY)
    mark("est1", main)
    mark("attn0", main)
    _abi.layer_attention(q, k, v, out, plan.heads, idx=idx, cnt=cnt,
                         idx_slots=len(plan.block_heads), topk_max=plan.topk_max, ws=ws,
                         staged=True)
    mark("attn0_end", main)


_SIDE_STREAMS: Dict[int, "torch.cuda.Stream"] = {}


def _side_stream(device: torch.device) -> "torch.cuda.Stream":
    """The per-device side stream (default priority, created once): in layers
    with vertical_and_slash heads the K/V staging runs on it beside the
    estimators."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    st = _SIDE_STREAMS.get(index)
    if st is None:
        st = torch.cuda.Stream(device=torch.device("cuda", index))
        _SIDE_STREAMS[index] = st
    return st


def run_decode_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: torch.Tensor,
                         scale: float) -> torch.Tensor:
    """Decode launch: q [B, H, 1, D] against the whole cache k/v [B, H_kv, S_k, D]
    (the reference's decode_dense, backend_npu/attention.py:274-314)."""
    _abi.require_device(q, k, v)
    _abi.decode_attention(q, k, v, out, scale)
    return out


def init_minference_parameters(self) -> None:
    """Per-layer one-time setup (reference :175-213): reads starting_layer,
    is_search, config_path and the attn type injected by the patch, and loads
    this layer's patterns."""
    if getattr(self, "_minference_initialized", False):
        return
    config = self.config.to_dict()
    self.starting_layer = config.get("starting_layer", 0)
    self.is_search = config.get("is_search", False)
    self.config_path = config.get("config_path", "")
    self._minference_attn_type = config.get("minference_attn_type", "minference")
    self.best_pattern = load_layer_patterns(self.config_path, self.layer_idx)
    self._minference_plans = {}
    self._minference_initialized = True


def _layer_plan(self, n_heads: int, head_dim: int, s_k: int) -> LayerPlan:
    key = (n_heads, head_dim, s_k)
    plan = self._minference_plans.get(key)
    if plan is None:
        plan = build_layer_plan(self.best_pattern, n_heads, head_dim, s_k, self.layer_idx)
        self._minference_plans[key] = plan
    return plan


def _apply_rope(self, q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
    """RoPE of the layer's fresh q/k projections (reference :205-212, :336-341).

    On the GPU the one-pass HIP kernel rotates q and k in place (they are
    views of this forward's own projection outputs), bit-identical to the
    model's eager function.  Other inputs (CPU tensors of the host-side
    tests, tables the kernel does not take) go to the model module's
    ``apply_rotary_pos_emb``."""
    if rope_supported(q, k, cos, sin):
        return apply_rotary_pos_emb_gpu(q, k, cos, sin, inplace=True)
    from importlib import import_module

    rope = getattr(import_module(self.__class__.__module__), "apply_rotary_pos_emb")
    return rope(q, k, cos, sin)


def minference_forward():
    """Returns the forward bound onto each attention module by the patch."""

    def forward(
        self,
        hidden_states: torch.Tensor,
        position_embeddings: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
        attention_mask: Optional[torch.Tensor] = None,
        past_key_values=None,
        **kwargs,
    ):
        if past_key_values is None:
            past_key_values = kwargs.pop("past_key_value", None)
        self.init_minference_parameters()
        cfg = self.config
        bsz, q_len, _ = hidden_states.shape
        n_heads = cfg.num_attention_heads
        n_kv = cfg.num_key_value_heads
        hd = self.head_dim

        if "q_proj" in self._modules:
            query = self.q_proj(hidden_states)
            key = self.k_proj(hidden_states)
            value = self.v_proj(hidden_states)
        else:
            qkv = self.qkv_proj(hidden_states)
            qp = n_heads * hd
            kp = n_kv * hd
            query, key, value = qkv[..., :qp], qkv[..., qp:qp + kp], qkv[..., qp + kp:]
        query = query.view(bsz, q_len, n_heads, hd).transpose(1, 2)
        key = key.view(bsz, q_len, n_kv, hd).transpose(1, 2)
        value = value.view(bsz, q_len, n_kv, hd).transpose(1, 2)

        if position_embeddings is None:
            position_embeddings = kwargs.get("position_embeddings")
        if position_embeddings is None:
            raise ValueError("position_embeddings (cos, sin) are required")
        cos, sin = position_embeddings
        query, key = _apply_rope(self, query, key, cos, sin)

        if past_key_values is not None and hasattr(past_key_values, "update"):
            key, value = past_key_values.update(key, value, self.layer_idx)

        if self.is_search:
            # reference :374-382 warns and :392-396 runs the layer dense
            warnings.warn("is_search=True: no pattern search runs; the layer runs dense "
                          "attention", stacklevel=2)

        # output written in [B, S, H, D] order; the kernel sees a [B, H, S, D] view
        out_bshd = torch.empty((bsz, q_len, n_heads, hd), dtype=query.dtype,
                               device=query.device)
        out = out_bshd.transpose(1, 2)
        if q_len == 1:
            # decode: one query row sees the whole cache (reference :488-490)
            run_decode_attention(query, key, value, out, dense_scale(hd))
        else:
            if (self._minference_attn_type == "dense" or self.layer_idx < self.starting_layer
                    or self.is_search):
                plan = dense_plan(n_heads, hd)
            else:
                plan = _layer_plan(self, n_heads, hd, key.shape[2])
            run_layer_attention(query, key, value, plan, out)

        attn_output = out_bshd.reshape(bsz, q_len, n_heads * hd)
        attn_output = self.o_proj(attn_output)
        return attn_output, None

    return forward

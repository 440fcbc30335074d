"""Weight provider over NF4 shards: the seam between the shard loader and the
trainer (doublepass/src/weight_provider.rs:33-52, shard_provider.rs:12-148).

``ShardEngineProvider.load_layer_weights`` keeps the reference's behaviour
(every parameter as fp32 values of its f16 load_param result,
shard_provider.rs:50-64,103-130), but on the device; ``load_layer_nf4``
is the drop-in the fused GEMM consumes: NF4 parameters stay packed on the
device (no f16/f32 widening), other parameters come back as f16.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, Optional

import torch

from .shard import MalformedIndexEntry, ShardEngineError, ShardLoader


class ProviderError(Exception):
    """weight_provider.rs:10-24."""


class ProviderIoError(ProviderError):
    """ProviderError::IoError."""


class ProviderNotFound(ProviderError):
    """ProviderError::NotFound."""


class ProviderConversionError(ProviderError):
    """ProviderError::ConversionError."""


class ParamNameMap:
    """shard_provider.rs:16-47."""

    def __init__(self, field_to_suffix: Dict[str, str], layer_prefix: str):
        self.field_to_suffix = dict(field_to_suffix)
        self.layer_prefix = layer_prefix

    @classmethod
    def llama(cls) -> "ParamNameMap":
        return cls({
            "rms1_w": "input_layernorm.weight",
            "wq": "self_attn.q_proj.weight",
            "wk": "self_attn.k_proj.weight",
            "wv": "self_attn.v_proj.weight",
            "wo": "self_attn.o_proj.weight",
            "rms2_w": "post_attention_layernorm.weight",
            "wg": "mlp.gate_proj.weight",
            "wu": "mlp.up_proj.weight",
            "wd": "mlp.down_proj.weight",
        }, "model.layers")

    def param_key(self, layer_idx: int, field: str) -> Optional[str]:
        suffix = self.field_to_suffix.get(field)
        if suffix is None:
            return None
        return f"{self.layer_prefix}.{layer_idx}.{suffix}"


FIELDS = ("rms1_w", "wq", "wk", "wv", "wo", "rms2_w", "wg", "wu", "wd")


class ShardEngineProvider:
    """shard_provider.rs:70-148 with the weights kept on the device."""

    def __init__(self, model_dir, param_map: ParamNameMap, num_layers: int, d_model: int,
                 d_ff: int, n_heads: int):
        try:
            self.loader = ShardLoader(model_dir)
        except ShardEngineError as e:
            raise ProviderIoError(str(e)) from None
        self.param_map = param_map
        self._num_layers, self._d_model, self._d_ff, self._n_heads = (
            num_layers, d_model, d_ff, n_heads)

    def _key(self, layer_idx: int, field: str) -> str:
        key = self.param_map.param_key(layer_idx, field)
        if key is None:
            raise ProviderNotFound(field)
        return key

    def load_layer_weights(self, layer_idx: int, cfg=None) -> Dict[str, torch.Tensor]:
        """shard_provider.rs:103-130: each field as fp32 values of the f16
        load_param bytes (exact widening, shard_provider.rs:50-64)."""
        out = {}
        for f in FIELDS:
            try:
                out[f] = self.loader.load_param_device(self._key(layer_idx, f)).float()
            except ShardEngineError as e:
                raise ProviderIoError(str(e)) from None
        return out

    def load_layer_nf4(self, layer_idx: int) -> Dict[str, object]:
        """NF4 fields as device Nf4Weight (packed payload, no widening); the
        others as float16 device tensors."""
        out = {}
        for f in FIELDS:
            key = self._key(layer_idx, f)
            try:
                info = self.loader.param_info(key)
                if info.precision != 0:
                    out[f] = self.loader.load_param_nf4(key)
                else:
                    out[f] = self.loader.load_param_device(key)
            except ShardEngineError as e:
                raise ProviderIoError(str(e)) from None
        return out

    def num_layers(self) -> int:
        return self._num_layers

    def d_model(self) -> int:
        return self._d_model

    def d_ff(self) -> int:
        return self._d_ff

    def n_heads(self) -> int:
        return self._n_heads

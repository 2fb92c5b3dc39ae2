"""The sparse attention layer as the opaque torch operator ``semblo::attention``.

Same schema, dispatch keys and layer lookup as the reference's operator
(semblo/vllm_plugin/attention_op.py:94-120): the caller owns every tensor,
the operator writes ``output`` in place and returns nothing, and the layer is
reached by name through a table.  ROCm's torch maps HIP devices to the CUDA
dispatch key.  The CPU key raises: this build runs on the GPU only.
"""
from __future__ import annotations

from typing import Any

import torch

_OP_NAMESPACE = "semblo"
_OP_NAME = "attention"
SPLITTING_OP_NAME = f"{_OP_NAMESPACE}::{_OP_NAME}"

_LAYERS: dict[str, Any] = {}


def register_layer(layer_name: str, layer: Any) -> None:
    _LAYERS[str(layer_name)] = layer


def registered_layer(layer_name: str) -> Any:
    layer = _LAYERS.get(str(layer_name))
    if layer is None:
        raise RuntimeError(f"layer name {layer_name!r} is unknown to semblo::attention: "
                           "construct its SembloAttention (which calls register_layer) first")
    return layer


def _attention(positions, hidden_states, q_post, k_post, v_states, q_pre, k_pre, output,
               layer_name) -> None:
    registered_layer(layer_name).attention_forward(
        positions, hidden_states, q_post, k_post, v_states, q_pre, k_pre, output)


def _attention_cpu(*args) -> None:
    raise RuntimeError("semblo::attention runs on the GPU only (the HIP kernels have no CPU path)")


def _attention_fake(positions, hidden_states, q_post, k_post, v_states, q_pre, k_pre, output,
                    layer_name) -> None:
    return None


_LIBRARY: torch.library.Library | None = None


def _register() -> None:
    global _LIBRARY
    if _LIBRARY is not None:
        return
    library = torch.library.Library(_OP_NAMESPACE, "FRAGMENT")
    library.define(
        f"{_OP_NAME}(Tensor positions, Tensor hidden_states, "
        "Tensor q_post, Tensor? k_post, Tensor? v_states, "
        "Tensor q_pre, Tensor? k_pre, "
        "Tensor(a!) output, str layer_name) -> ()")
    library.impl(_OP_NAME, _attention_cpu, "CPU")
    library.impl(_OP_NAME, _attention, "CUDA")
    library._register_fake(_OP_NAME, _attention_fake)
    _LIBRARY = library


_register()
sparse_attention_op = getattr(torch.ops, _OP_NAMESPACE).attention

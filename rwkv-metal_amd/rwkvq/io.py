"""Packed-checkpoint I/O: quantized models in MLX's on-disk form.

    save_quantized(model, path)        <- model.save_weights of an nn.quantize'd MLX model
    load_quantized(model, path)        <- nn.quantize(model, class_predicate=lambda p, m:
                                          f"{p}.scales" in weights) + model.load_weights

A quantized module is stored under its module path as `<path>.weight` (the
packed words, uint32), `<path>.scales`, `<path>.biases` and, for a Linear
with a bias, `<path>.bias` -- the parameter names MLX's QuantizedLinear /
QuantizedEmbedding save (rwkv_metal/lora/finetune.py:88-89 quantizes with
nn.quantize; the same names are the packed checkpoint's keys).  Every other
tensor of the state dict is stored as it is.  The file's metadata carries
{"format": "mlx", "quantization": {"group_size", "bits", per-module
overrides}}, the quantization entry of an MLX model config.

Loading needs no quantization arithmetic: the modules that have a
`<path>.scales` tensor in the file are replaced by empty quantized modules
whose bits and group size follow from the stored shapes (bits = 32 * words
per row / in_features, group_size = in_features / groups per row), and the
tensors are then copied in.  LoRA adapters are saved and loaded separately
(rwkvq.lora.save_lora / load_lora, rwkv_metal/lora/lora.py:136-148).
"""
from __future__ import annotations

import json
from typing import Dict, Optional

import torch
from torch import Tensor, nn

from .nn import QuantizedEmbedding, QuantizedLinear


def _quantized_modules(model: nn.Module):
    for path, m in model.named_modules():
        if isinstance(m, (QuantizedLinear, QuantizedEmbedding)):
            yield path, m


def save_quantized(model: nn.Module, path: str, metadata: Optional[Dict[str, str]] = None) -> None:
    """Write model.state_dict() to `path` (safetensors), packed words as uint32."""
    from safetensors.torch import save_file

    qpaths = {p for p, _ in _quantized_modules(model)}
    tensors = {}
    for k, v in model.state_dict().items():
        t = v.detach().contiguous().cpu()
        mod, _, leaf = k.rpartition(".")
        if leaf == "weight" and mod in qpaths:
            t = t.view(torch.uint32)
        tensors[k] = t
    settings = {p: {"group_size": m.group_size, "bits": m.bits}
                for p, m in _quantized_modules(model)}
    quant = {}
    if settings:
        first = next(iter(settings.values()))
        quant = dict(first)
        for p, s in settings.items():
            if s != first:
                quant[p] = s
    meta = {"format": "mlx", "quantization": json.dumps(quant)}
    meta.update(metadata or {})
    save_file(tensors, path, metadata=meta)


def _empty_quantized(module: nn.Module, words: Tensor, scales: Tensor, has_bias: bool
                     ) -> nn.Module:
    if isinstance(module, nn.Linear):
        in_f, out_f = module.in_features, module.out_features
    elif isinstance(module, nn.Embedding):
        out_f, in_f = module.num_embeddings, module.embedding_dim
    elif isinstance(module, (QuantizedLinear, QuantizedEmbedding)):
        return module
    else:
        raise TypeError(f"cannot load packed weights into {type(module).__name__}")
    if words.shape[0] != out_f or scales.shape[0] != out_f:
        raise ValueError(f"packed rows {words.shape[0]} do not match the module's {out_f}")
    bits, rem = divmod(words.shape[1] * 32, in_f)
    if rem or scales.shape[1] == 0 or in_f % scales.shape[1]:
        raise ValueError(f"packed shapes {tuple(words.shape)} / {tuple(scales.shape)} do not "
                         f"fit in_features {in_f}")
    gs = in_f // scales.shape[1]
    dev = next((t.device for t in module.parameters()), torch.device("cpu"))
    if isinstance(module, nn.Linear):
        return QuantizedLinear(in_f, out_f, bias=has_bias, group_size=gs, bits=bits, device=dev,
                               dtype=scales.dtype)
    return QuantizedEmbedding(out_f, in_f, group_size=gs, bits=bits, device=dev,
                              dtype=scales.dtype)


def load_quantized(model: nn.Module, path: str, strict: bool = True) -> nn.Module:
    """Load a checkpoint written by save_quantized (or by MLX for a quantized
    model): quantize the modules the file holds packed, then copy every tensor."""
    from safetensors.torch import load_file

    weights = load_file(path)
    for mpath in sorted({k[: -len(".scales")] for k in weights if k.endswith(".scales")}):
        parent_path, _, name = mpath.rpartition(".")
        parent = model.get_submodule(parent_path) if parent_path else model
        child = getattr(parent, name)
        setattr(parent, name, _empty_quantized(child, weights[f"{mpath}.weight"],
                                               weights[f"{mpath}.scales"],
                                               f"{mpath}.bias" in weights))
    state = model.state_dict()
    for k, v in weights.items():
        if k in state and state[k].dtype == torch.int32 and v.dtype == torch.uint32:
            weights[k] = v.view(torch.int32)
    missing, unexpected = model.load_state_dict(weights, strict=False)
    if strict and (missing or unexpected):
        raise KeyError(f"checkpoint mismatch: missing {sorted(missing)}, "
                       f"unexpected {sorted(unexpected)}")
    return model


def quantization_config(path: str) -> dict:
    """The {"group_size", "bits", per-module overrides} entry of a saved checkpoint."""
    from safetensors import safe_open

    with safe_open(path, "pt") as f:
        meta = f.metadata() or {}
    return json.loads(meta.get("quantization", "{}"))

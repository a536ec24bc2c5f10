"""Quantized modules with MLX's parameter layout (weight / scales / biases).

    QuantizedLinear(input_dims, output_dims, bias, group_size, bits)   <- mlx.nn.QuantizedLinear
    QuantizedLinear.from_linear(linear, group_size, bits)              <- .from_linear
    QuantizedEmbedding(num_embeddings, dims, group_size, bits)         <- mlx.nn.QuantizedEmbedding
    quantize(model, group_size, bits, class_predicate)                 <- mlx.nn.quantize

Reference call sites: rwkv_metal/lora/finetune.py:88-89 (nn.quantize with a
path predicate), rwkv_metal/lora/lora.py:45-46 (QuantizedLinear.from_linear),
the model's projections rwkv_metal/model/rwkv7_x070.py:108-111,215-216,262-266.

State-dict keys are `weight` (packed words, int32 holding the uint32 bits),
`scales`, `biases` and optionally `bias` -- the names MLX saves, so packed
checkpoints map key for key.  The quantized tensors are buffers: the base is
frozen, as MLX's QuantizedLinear freezes itself.
"""
from __future__ import annotations

from typing import Callable, Optional, Union

import torch
from torch import Tensor, nn

from . import ops


class QuantizedLinear(nn.Module):
    """y = x @ dequant(weight)^T (+ bias), evaluated by the packed-weight kernels."""

    def __init__(self, input_dims: int, output_dims: int, bias: bool = True,
                 group_size: int = 64, bits: int = 4, device=None,
                 dtype: torch.dtype = torch.bfloat16):
        super().__init__()
        ops._check_args(group_size, bits)
        if input_dims % group_size:
            raise ValueError(f"input_dims {input_dims} not divisible by group_size {group_size}")
        self.group_size, self.bits = group_size, bits
        self.in_features, self.out_features = input_dims, output_dims
        self.register_buffer("weight", torch.zeros(output_dims, input_dims * bits // 32,
                                                   dtype=torch.int32, device=device))
        self.register_buffer("scales", torch.zeros(output_dims, input_dims // group_size,
                                                   dtype=dtype, device=device))
        self.register_buffer("biases", torch.zeros_like(self.scales))
        if bias:
            self.register_buffer("bias", torch.zeros(output_dims, dtype=dtype, device=device))
        else:
            self.bias = None

    @classmethod
    def from_linear(cls, linear: nn.Linear, group_size: int = 64, bits: int = 4
                    ) -> "QuantizedLinear":
        out_f, in_f = linear.weight.shape
        w = linear.weight.detach()
        q = cls.__new__(cls)
        nn.Module.__init__(q)
        ops._check_args(group_size, bits)
        q.group_size, q.bits = group_size, bits
        q.in_features, q.out_features = in_f, out_f
        wq, s, b = ops.quantize(w, group_size, bits)
        q.register_buffer("weight", wq)
        q.register_buffer("scales", s)
        q.register_buffer("biases", b)
        if linear.bias is not None:
            q.register_buffer("bias", linear.bias.detach().clone())
        else:
            q.bias = None
        return q

    def forward(self, x: Tensor) -> Tensor:
        y = ops.quantized_matmul(x, self.weight, self.scales, self.biases, True,
                                 self.group_size, self.bits)
        if self.bias is not None:
            y = y + self.bias
        return y

    def dequantized_weight(self) -> Tensor:
        return ops.dequantize(self.weight, self.scales, self.biases, self.group_size, self.bits)

    def extra_repr(self) -> str:
        return (f"input_dims={self.in_features}, output_dims={self.out_features}, "
                f"bias={self.bias is not None}, group_size={self.group_size}, bits={self.bits}")


class QuantizedEmbedding(nn.Module):
    """nn.QuantizedEmbedding: a [num_embeddings, dims] table in packed form;
    the lookup is one fused gather-dequantize launch (rq_embedding)."""

    def __init__(self, num_embeddings: int, dims: int, group_size: int = 64, bits: int = 4,
                 device=None, dtype: torch.dtype = torch.bfloat16):
        super().__init__()
        ops._check_args(group_size, bits)
        if dims % group_size:
            raise ValueError(f"dims {dims} not divisible by group_size {group_size}")
        self.group_size, self.bits = group_size, bits
        self.num_embeddings, self.dims = num_embeddings, dims
        self.register_buffer("weight", torch.zeros(num_embeddings, dims * bits // 32,
                                                   dtype=torch.int32, device=device))
        self.register_buffer("scales", torch.zeros(num_embeddings, dims // group_size,
                                                   dtype=dtype, device=device))
        self.register_buffer("biases", torch.zeros_like(self.scales))

    @classmethod
    def from_embedding(cls, emb: nn.Embedding, group_size: int = 64, bits: int = 4
                       ) -> "QuantizedEmbedding":
        n, d = emb.weight.shape
        q = cls.__new__(cls)
        nn.Module.__init__(q)
        ops._check_args(group_size, bits)
        q.group_size, q.bits, q.num_embeddings, q.dims = group_size, bits, n, d
        wq, s, b = ops.quantize(emb.weight.detach(), group_size, bits)
        q.register_buffer("weight", wq)
        q.register_buffer("scales", s)
        q.register_buffer("biases", b)
        return q

    def forward(self, idx: Tensor) -> Tensor:
        return ops.quantized_embedding(idx, self.weight, self.scales, self.biases,
                                       self.group_size, self.bits)

    def as_linear(self, x: Tensor) -> Tensor:
        """Tied output head: x @ dequant(weight)^T."""
        return ops.quantized_matmul(x, self.weight, self.scales, self.biases, True,
                                    self.group_size, self.bits)


Predicate = Callable[[str, nn.Module], Union[bool, dict]]


def is_quantizable(module: nn.Module) -> bool:
    """Modules the quantizer knows how to convert (MLX: hasattr(m, 'to_quantized'))."""
    return isinstance(module, (nn.Linear, nn.Embedding)) or hasattr(module, "to_quantized")


def _to_quantized(module: nn.Module, group_size: int, bits: int) -> nn.Module:
    if hasattr(module, "to_quantized"):
        return module.to_quantized(group_size=group_size, bits=bits)
    if isinstance(module, nn.Linear):
        return QuantizedLinear.from_linear(module, group_size, bits)
    if isinstance(module, nn.Embedding):
        return QuantizedEmbedding.from_embedding(module, group_size, bits)
    raise TypeError(f"cannot quantize {type(module).__name__}")


def quantize(model: nn.Module, group_size: int = 64, bits: int = 4,
             class_predicate: Optional[Predicate] = None) -> nn.Module:
    """In-place swap of the selected submodules for quantized ones (mlx.nn.quantize).

    class_predicate(path, module) returns False (skip), True (use group_size/bits)
    or a dict with per-module 'group_size'/'bits' -- the way mixed bit widths
    (e.g. a 3-bit body with an 8-bit head) are expressed.  The default selects
    every quantizable module whose last dimension divides by group_size.
    """
    if class_predicate is None:
        def class_predicate(path, m):
            return is_quantizable(m) and m.weight.shape[-1] % group_size == 0

    def visit(parent: nn.Module, prefix: str) -> None:
        for name, child in list(parent.named_children()):
            path = f"{prefix}.{name}" if prefix else name
            sel = class_predicate(path, child)
            if sel:
                gs = sel.get("group_size", group_size) if isinstance(sel, dict) else group_size
                b = sel.get("bits", bits) if isinstance(sel, dict) else bits
                setattr(parent, name, _to_quantized(child, gs, b))
            else:
                visit(child, path)

    visit(model, "")
    return model

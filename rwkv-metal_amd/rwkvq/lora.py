"""LoRA / QLoRA layer on a frozen quantized base, with the reference's API.

    LoRALinear(linear, rank, alpha, dropout, quantize_base, q_group_size,
               base_module, dtype)                       <- rwkv_metal/lora/lora.py:24-67
    add_lora(model, rank, alpha, dropout, tmix_targets, cmix_targets,
             quantize_base, q_group_size, layers)        <- rwkv_metal/lora/lora.py:74-108
    quantize_base_model(model, bits, group_size, targets) <- rwkv_metal/lora/finetune.py:70-91
    BIG_QUANT_TARGETS                                     <- rwkv_metal/lora/finetune.py:42
    lora_state / save_lora / load_lora / merge_lora       <- rwkv_metal/lora/lora.py:132-172

y = base(x) + (alpha/rank) * (x @ A^T) @ B^T with A ~ N(0, 1)/sqrt(in_features)
and B = 0 (lora.py:54-56).  Only lora_a / lora_b are trainable (lora.py:101-102).
Over a QuantizedLinear base with bf16 or fp32 activations (bf16 adapters)
the low-rank term is fused into the packed-weight GEMMs, forward and dX
(rq_qlora / rq_qlora_dx / rq_qmm_lora, _QLoRAFunction); other bases and
dtypes compose the ops.
The model layout is the reference's: model.blocks[i].tmix.{r,k,v,o}_proj and
model.blocks[i].cmix.{key,value}.

merge_lora differs on purpose: the reference adds the float delta to the
packed words of a quantized base (lora.py:65-67), which yields garbage; here a
quantized base is refused unless requantize=True, which dequantizes, adds the
delta and quantizes again with the base's group size and bits.
"""
from __future__ import annotations

import math
from typing import Iterable, Optional, Tuple

import torch
from torch import Tensor, nn

from . import ops
from .nn import QuantizedEmbedding, QuantizedLinear, is_quantizable
from .nn import quantize as nn_quantize

BIG_QUANT_TARGETS = ("cmix.key", "cmix.value", "head", "emb")
TMIX_TARGETS = ("r_proj", "k_proj", "v_proj", "o_proj")
CMIX_TARGETS = ("key", "value")


def _promote(a: torch.dtype, b: torch.dtype) -> torch.dtype:
    return a if a == b else torch.float32


class _QLoRAFunction(torch.autograd.Function):
    """y = base(x) + scale * (x A^T) B^T over a QuantizedLinear base with the
    low-rank term fused into the packed-weight GEMMs.  Rank 16 at 4 or 8 bits
    (rq_qlora): the forward is one launch that also computes z = x A^T
    inside the transpose=True GEMM and adds z B^T in its output stage; dX is
    one launch (rq_qlora_dx) that computes u = dY B inside the
    transpose=False GEMM and adds scale * u A, reading A and B as stored; dA =
    scale * u^T x and dB = scale * dY^T z are one rq_lora_grads launch.  Other ranks run z and u as rq_lora_down launches
    and the term with rq_qmm_lora.  The frozen base gets no gradient.

    fp32 x (the reference's default activations) is rounded to bf16 once, by
    one cast, and so is fp32 dY: every kernel rounds its fp32 operands to bf16
    as it stages them anyway (the results are the bits the fp32 inputs give),
    but the GEMMs re-read their activation tiles once per column tile, so
    twice the bytes per re-read cost more than the cast.  y and dX stay fp32,
    and x is saved for the backward in bf16."""

    @staticmethod
    def forward(ctx, x2, lora_a, lora_b, base, scale):
        gs, bits = base.group_size, base.bits
        xdt = x2.dtype
        xb = x2.to(torch.bfloat16) if xdt == torch.float32 else x2
        yz = ops.qlora_fused(xb, base.weight, base.scales, base.biases, lora_a, lora_b, scale,
                             True, gs, bits, out_dtype=ops._promote(xdt, base.scales.dtype))
        if yz is not None:
            y, z = yz      # one launch: z = x A^T inside the GEMM
        else:
            z = ops.lora_down(x2, lora_a)
            y = ops.quantized_matmul_lora(x2, base.weight, base.scales, base.biases, z, lora_b,
                                          scale, True, gs, bits)
        ctx.save_for_backward(xb, z, lora_a, lora_b)
        ctx.base, ctx.scale, ctx.xdt = base, scale, xdt
        return y

    @staticmethod
    def backward(ctx, dy):
        xb, z, lora_a, lora_b = ctx.saved_tensors
        base, scale, xdt = ctx.base, ctx.scale, ctx.xdt
        gs, bits = base.group_size, base.bits
        dy = dy.contiguous().to(xdt)
        dyb = dy.to(torch.bfloat16) if xdt == torch.float32 else dy
        dx = da = db = None
        dxu = None
        if ctx.needs_input_grad[0]:
            # one launch from the adapters as stored: u = dY B inside the GEMM
            dxu = ops.qlora_dx_fused(dyb, base.weight, base.scales, base.biases, lora_a, lora_b,
                                     scale, gs, bits, out_dtype=ops._promote(xdt, base.scales.dtype))
            if dxu is not None:
                dx, u = dxu
            else:
                bt = lora_b.t().contiguous()
                u = ops.lora_down(dy, bt)
                dx = ops.quantized_matmul_lora(dy, base.weight, base.scales, base.biases, u,
                                               lora_a.t().contiguous(), scale, False, gs, bits)
            dx = dx.to(xdt)
        else:
            u = ops.lora_down(dyb, lora_b.t().contiguous())
        # both adapter gradients in one launch, fp32 accumulation, one rounding
        want_a, want_b = ctx.needs_input_grad[1], ctx.needs_input_grad[2]
        da, db = ops.lora_grads(xb if want_a else None, u if want_a else None,
                                dyb if want_b else None, z if want_b else None, scale)
        if da is not None:
            da = da.to(lora_a.dtype)
        if db is not None:
            db = db.to(lora_b.dtype)
        return dx, da, db, None, None


class LoRALinear(nn.Module):
    """Frozen base (bf16 Linear, QuantizedLinear, or any module with
    out_features/in_features/__call__) plus a trainable low-rank update."""

    def __init__(self, linear: Optional[nn.Linear] = None, rank: int = 16, alpha: float = 32.0,
                 dropout: float = 0.0, quantize_base: int = 0, q_group_size: int = 64,
                 base_module: Optional[nn.Module] = None, dtype: Optional[torch.dtype] = None):
        super().__init__()
        if base_module is not None:
            out_features, in_features = base_module.out_features, base_module.in_features
            dtype = dtype or torch.bfloat16
            device = next((t.device for t in base_module.buffers()), None) or next(
                (t.device for t in base_module.parameters()), torch.device("cpu"))
            self.linear = base_module
        else:
            out_features, in_features = linear.weight.shape
            dtype = linear.weight.dtype
            device = linear.weight.device
            if quantize_base:
                self.linear = QuantizedLinear.from_linear(linear, group_size=q_group_size,
                                                          bits=quantize_base)
            else:
                self.linear = linear
        self.in_features, self.out_features = in_features, out_features
        self.rank = rank
        self.scale = alpha / rank
        self.dropout = nn.Dropout(dropout) if dropout > 0 else None
        scale_a = 1.0 / math.sqrt(in_features)
        self.lora_a = nn.Parameter(
            (torch.randn(rank, in_features, device=device) * scale_a).to(dtype))
        self.lora_b = nn.Parameter(torch.zeros(out_features, rank, device=device, dtype=dtype))

    def _fusable(self, x: Tensor) -> bool:
        """The low-rank term can ride on the packed-weight GEMMs: quantized
        base, bf16 adapters, a supported rank, no active dropout on z (its
        mask would have to be saved for the backward), and bf16 activations
        or fp32 ones (the reference's default residual stream,
        rwkv_metal/model/rwkv7_x070.py:51,189-194), which the kernels round to
        bf16 as they stage them; y and dX are then fp32."""
        return (isinstance(self.linear, QuantizedLinear) and x.is_cuda
                and x.dtype in (torch.bfloat16, torch.float32)
                and self.lora_a.dtype == self.lora_b.dtype == torch.bfloat16
                and self.rank in (16, 32, 48, 64)
                and (self.dropout is None or not self.training))

    def forward(self, x: Tensor) -> Tensor:
        if self._fusable(x):
            lead = x.shape[:-1]
            x2 = x.reshape(-1, x.shape[-1]).contiguous()
            y = _QLoRAFunction.apply(x2, self.lora_a, self.lora_b, self.linear, self.scale)
            if self.linear.bias is not None:
                y = y + self.linear.bias
            return y.reshape(*lead, y.shape[-1])
        base = self.linear(x)
        ct = _promote(x.dtype, self.lora_a.dtype)
        z = x.to(ct) @ self.lora_a.to(ct).t()
        if self.dropout is not None:
            z = self.dropout(z)
        return base + self.scale * (z @ self.lora_b.to(ct).t())

    def merged_weight(self, requantize: bool = False):
        delta = self.scale * (self.lora_b.float() @ self.lora_a.float())
        if isinstance(self.linear, QuantizedLinear):
            if not requantize:
                raise ValueError(
                    "cannot add a float delta to a quantized base (its weight holds packed "
                    "codes); pass requantize=True to dequantize, merge and quantize again")
            w = self.linear.dequantized_weight().float() + delta
            return w.to(self.linear.scales.dtype)
        w = self.linear.weight
        return w + delta.to(w.dtype)


def _blocks(model):
    return model.blocks


def add_lora(model: nn.Module, rank: int = 16, alpha: float = 32.0, dropout: float = 0.0,
             tmix_targets=TMIX_TARGETS, cmix_targets=(), quantize_base: int = 0,
             q_group_size: int = 64, layers: Optional[Iterable[int]] = None):
    """Wrap the target Linears of the selected blocks in LoRALinear and freeze
    everything but the adapters.  quantize_base: 0 keeps the base as is; 2-8
    quantizes it (QLoRA)."""
    wrapped = []

    def mk(mod):
        return LoRALinear(mod, rank, alpha, dropout, quantize_base, q_group_size)

    blocks = _blocks(model)
    n_layer = len(blocks)
    sel = set(range(n_layer)) if layers is None else set(i % n_layer for i in layers)
    for li, blk in enumerate(blocks):
        if li not in sel:
            continue
        for name in tmix_targets:
            mod = getattr(blk.tmix, name, None)
            if isinstance(mod, nn.Linear):
                setattr(blk.tmix, name, mk(mod))
                wrapped.append(f"tmix.{name}")
        for name in cmix_targets:
            mod = getattr(blk.cmix, name, None)
            if isinstance(mod, nn.Linear):
                setattr(blk.cmix, name, mk(mod))
                wrapped.append(f"cmix.{name}")

    for p in model.parameters():
        p.requires_grad_(False)
    _unfreeze_adapters(model)

    info = _param_stats(model)
    info["wrapped_per_block"] = sorted(set(wrapped))
    info["num_adapters"] = len(wrapped)
    return model, info


def _unfreeze_adapters(model: nn.Module) -> None:
    for m in model.modules():
        if isinstance(m, LoRALinear):
            m.lora_a.requires_grad_(True)
            m.lora_b.requires_grad_(True)


def _param_stats(model: nn.Module) -> dict:
    total = sum(p.numel() for p in model.parameters())
    # packed quantized tensors count as parameters, as in MLX's parameter tree
    for m in model.modules():
        if isinstance(m, (QuantizedLinear, QuantizedEmbedding)):
            total += m.weight.numel() + m.scales.numel() + m.biases.numel()
    train = sum(p.numel() for p in model.parameters() if p.requires_grad)
    return {"total_params": total, "trainable_params": train,
            "trainable_pct": 100.0 * train / max(1, total)}


def lora_state(model: nn.Module) -> dict:
    return {k: v for k, v in model.named_parameters() if v.requires_grad}


def save_lora(model: nn.Module, path: str) -> None:
    from safetensors.torch import save_file
    save_file({k: v.detach().contiguous().cpu() for k, v in lora_state(model).items()}, path)


def load_lora(model: nn.Module, path: str) -> nn.Module:
    from safetensors.torch import load_file
    weights = load_file(path)
    params = dict(model.named_parameters())
    for k, v in weights.items():
        if k not in params:
            raise KeyError(f"adapter tensor {k} has no matching parameter")
        with torch.no_grad():
            params[k].copy_(v.to(params[k].device, params[k].dtype))
    return model


def merge_lora(model: nn.Module, requantize: bool = False) -> nn.Module:
    """Fold every LoRALinear back into its base (in place)."""
    def merged(child: LoRALinear) -> nn.Module:
        base = child.linear
        if isinstance(base, QuantizedLinear):
            w = child.merged_weight(requantize=requantize)
            lin = nn.Linear(base.in_features, base.out_features, bias=base.bias is not None,
                            device=w.device, dtype=w.dtype)
            with torch.no_grad():
                lin.weight.copy_(w)
                if base.bias is not None:
                    lin.bias.copy_(base.bias)
            return QuantizedLinear.from_linear(lin, base.group_size, base.bits)
        with torch.no_grad():
            base.weight.copy_(child.merged_weight())
        return base

    # refuse before mutating anything: a quantized base merges only by requantizing
    if not requantize:
        for m in model.modules():
            if isinstance(m, LoRALinear) and isinstance(m.linear, QuantizedLinear):
                m.merged_weight(requantize=False)  # raises ValueError

    def replace_in(parent: nn.Module) -> None:
        for cname, child in list(parent.named_children()):
            if isinstance(child, LoRALinear):
                setattr(parent, cname, merged(child))
            else:
                replace_in(child)

    replace_in(model)
    for p in model.parameters():
        p.requires_grad_(True)
    return model


def quantize_base_model(model: nn.Module, bits: int = 4, group_size: int = 64,
                        targets: Tuple[str, ...] = BIG_QUANT_TARGETS) -> nn.Module:
    """Quantize, in place, only the modules whose path ends with one of
    `targets` (cmix.key/value, head, emb by default)."""
    def predicate(path, module):
        return is_quantizable(module) and any(path.endswith(t) for t in targets)

    nn_quantize(model, group_size=group_size, bits=bits, class_predicate=predicate)
    return model

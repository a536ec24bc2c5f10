"""The .rwkvq (rwkv-quant "sb6") QLoRA base, with the reference's API.

    load_sidecar(path)                      <- rwkv_metal/lora/rwkvq_linear.py:85-103
    RwkvqLinear(qblk, qsqm, ddm, shape,
                gw_gs, gw_sb, xbits)        <- rwkvq_linear.py:106-179 (dense dequant + matmul)
    RwkvqNativeLinear(lin)                  <- rwkvq_native.py:93-122 (one-time repack into the
                                               MLX affine layout, then quantized_matmul)
    RwkvqHybridLinear(lin)                  <- rwkvq_hybrid.py:47-91 (repacked codes, scales and
                                               biases expanded from the compact form per call)
    add_lora_rwkvq(model, sidecar_path,...) <- add_rwkvq.py:40-102 (swap the projections, FFN
                                               and head for the sb6 base, LoRA on tmix targets)

Tensors are the K3-interleaved arrays of the sidecar that rwkv-quant's
export writes (`<path>.safetensors` with `<key>::qblk`, `<key>::qsqm`,
`<key>::ddm`, and `<path>.json` whose "tensors" entry gives each key's
shape, gw_gs, gw_sb and xbits).  Reading a `.rwkvq` container directly needs
rwkv_quant.formats.codec (open_rwkvq / sb6_to_k3, rwkvq_linear.py:63-83),
which is not part of this build: such paths raise.  Every computation runs in
librwkvq_hip.so (rq_sb6_dequantize, rq_sb6_to_affine, rq_qmm).
"""
from __future__ import annotations

import json
import os
from typing import Dict, Tuple

import torch
from torch import Tensor, nn

from . import ops
from .ops import _DeviceGuard, _stream_on
from ._lib import DTYPE_CODE, check, lib
from .lora import TMIX_TARGETS, LoRALinear, _param_stats, _unfreeze_adapters

GROUP_SIZE = 32  # rwkvq_native.py:45: the repacked layout's group size

_SIDECAR_CACHE: Dict[str, Tuple[dict, dict]] = {}
_TMIX_KEY = {"r_proj": "receptance", "k_proj": "key", "v_proj": "value", "o_proj": "output"}


def load_sidecar(path: str, device=None):
    """(arrays, manifest) of an exported sidecar `<path>.safetensors` +
    `<path>.json`; arrays are moved to `device` (default: the current GPU)."""
    key = (path, str(device))
    if key in _SIDECAR_CACHE:
        return _SIDECAR_CACHE[key]
    if path.endswith(".rwkvq") or not os.path.exists(path + ".safetensors"):
        raise NotImplementedError(
            f"{path}: reading a .rwkvq container needs rwkv_quant.formats.codec (open_rwkvq, "
            "sb6_to_k3), which this build does not include; export the sidecar "
            "(<path>.safetensors + <path>.json) and pass its path without the suffix")
    from safetensors.torch import load_file

    dev = device if device is not None else torch.device("cuda", torch.cuda.current_device())
    arrays = {k: v.to(dev) for k, v in load_file(path + ".safetensors").items()}
    with open(path + ".json") as f:
        manifest = json.load(f)
    _SIDECAR_CACHE[key] = (arrays, manifest)
    return arrays, manifest


def _dev_ptr(t: Tensor) -> int:
    return t.data_ptr() if t.numel() else 0


def _sb6_args(lin: "RwkvqLinear"):
    return (_dev_ptr(lin.qblk) or None, _dev_ptr(lin.qsqm), _dev_ptr(lin.ddm), lin.out_features,
            lin.in_features, lin.gw_gs, lin._gw_sb, lin.xbits)


def _to_affine(lin: "RwkvqLinear", codes: bool = True):
    """rq_sb6_to_affine: (w_q int32 [OUT, NB*bits] or None, scale f32, bias f32)."""
    ops._on_gpu(lin.qsqm)
    OUT, NB, bits = lin.out_features, lin.NB, 4 + lin.xbits
    dev = lin.qsqm.device
    wq = torch.empty(OUT, NB * bits, dtype=torch.int32, device=dev) if codes else None
    sc = torch.empty(OUT, NB, dtype=torch.float32, device=dev)
    bi = torch.empty_like(sc)
    with _DeviceGuard(dev):
        rc = lib().rq_sb6_to_affine(*_sb6_args(lin), _dev_ptr(wq) if codes else None,
                                    _dev_ptr(sc), _dev_ptr(bi),
                                    _stream_on(dev))
    check(rc, "sb6_to_affine")
    return wq, sc, bi


class RwkvqLinear(nn.Module):
    """Frozen linear over an sb6 tensor: y = x @ W^T with W dequantized on the
    fly each call (not kept dense; rwkvq_linear.py:106-112)."""

    def __init__(self, qblk: Tensor, qsqm: Tensor, ddm: Tensor, shape, gw_gs: int, gw_sb: int,
                 xbits: int):
        super().__init__()
        OUT, IN = shape
        if gw_gs != 32:
            raise ValueError(f"sb6 blocks are 32 codes (gw_gs={gw_gs})")
        self.out_features, self.in_features = OUT, IN
        self.NB, self.NSB = IN // gw_gs, IN // (gw_gs * gw_sb)
        self.gw_gs, self._gw_sb, self.xbits = gw_gs, gw_sb, xbits
        self.register_buffer("qblk", qblk.contiguous().view(torch.uint8).reshape(OUT, -1))
        self.register_buffer("qsqm", qsqm.contiguous().view(torch.uint8).reshape(OUT, -1))
        self.register_buffer("ddm", ddm.contiguous().view(torch.float16).reshape(OUT, -1))
        want = (OUT, self.NB * (16 + 4 * xbits)), (OUT, 2 * self.NB), (OUT, 2 * self.NSB)
        got = tuple(self.qblk.shape), tuple(self.qsqm.shape), tuple(self.ddm.shape)
        if got != want:
            raise ValueError(f"sb6 arrays have shapes {got}, expected {want}")

    @classmethod
    def from_sidecar(cls, sidecar_path: str, key: str, device=None) -> "RwkvqLinear":
        arrays, manifest = load_sidecar(sidecar_path, device)
        meta = manifest["tensors"][key]
        return cls(arrays[f"{key}::qblk"], arrays[f"{key}::qsqm"], arrays[f"{key}::ddm"],
                   tuple(meta["shape"]), meta["gw_gs"], meta["gw_sb"], meta["xbits"])

    def _dequant(self, dtype: torch.dtype) -> Tensor:
        ops._on_gpu(self.qblk)
        dev = self.qblk.device
        out = torch.empty(self.out_features, self.in_features, dtype=dtype, device=dev)
        with _DeviceGuard(dev):
            rc = lib().rq_sb6_dequantize(*_sb6_args(self), _dev_ptr(out), DTYPE_CODE[dtype],
                                         _stream_on(dev))
        check(rc, "sb6_dequantize")
        return out

    def _dequant_w(self) -> Tensor:
        """Dense bf16 weight (fp32 code*scale + min, rounded to bf16)."""
        return self._dequant(torch.bfloat16)

    def _dequant_w_fp32(self) -> Tensor:
        return self._dequant(torch.float32)

    def forward(self, x: Tensor) -> Tensor:
        w = self._dequant_w()
        ct = ops._promote(x.dtype, w.dtype)
        return x.to(ct) @ w.to(ct).t()


class RwkvqNativeLinear(nn.Module):
    """Frozen linear on the repacked sb6 data: y = quantized_matmul(x in fp32,
    w_q, scale, bias, transpose=True, group_size=32, bits=4+xbits) cast back
    to x's dtype.  The repack runs once, at construction."""

    def __init__(self, lin: RwkvqLinear):
        super().__init__()
        self.out_features, self.in_features = lin.out_features, lin.in_features
        self.bits = 4 + lin.xbits
        wq, sc, bi = _to_affine(lin)
        self.register_buffer("wq", wq)
        self.register_buffer("scale", sc)
        self.register_buffer("bias", bi)

    @classmethod
    def from_sidecar(cls, sidecar_path: str, key: str, device=None) -> "RwkvqNativeLinear":
        return cls(RwkvqLinear.from_sidecar(sidecar_path, key, device))

    def forward(self, x: Tensor) -> Tensor:
        return ops.quantized_matmul(x.float(), self.wq, self.scale, self.bias, True, GROUP_SIZE,
                                    self.bits).to(x.dtype)


class RwkvqHybridLinear(nn.Module):
    """Repacked codes plus the compact sb6 scales (qsqm, ddm), expanded to
    per-group fp32 scale/bias before every product (rwkvq_hybrid.py:47-91)."""

    def __init__(self, lin: RwkvqLinear):
        super().__init__()
        self.out_features, self.in_features = lin.out_features, lin.in_features
        self.NB, self.NSB, self._gw_sb = lin.NB, lin.NSB, lin._gw_sb
        self.gw_gs, self.xbits, self.bits = lin.gw_gs, lin.xbits, 4 + lin.xbits
        wq, _, _ = _to_affine(lin)
        self.register_buffer("wq", wq)
        self.register_buffer("qsqm", lin.qsqm)
        self.register_buffer("ddm", lin.ddm)
        self.register_buffer("qblk", torch.empty(0, dtype=torch.uint8, device=lin.qblk.device),
                             persistent=False)

    @classmethod
    def from_sidecar(cls, sidecar_path: str, key: str, device=None) -> "RwkvqHybridLinear":
        return cls(RwkvqLinear.from_sidecar(sidecar_path, key, device))

    def _expand_scale_bias(self):
        _, sc, bi = _to_affine(self, codes=False)
        return sc, bi

    def forward(self, x: Tensor) -> Tensor:
        sc, bi = self._expand_scale_bias()
        return ops.quantized_matmul(x.float(), self.wq, sc, bi, True, GROUP_SIZE,
                                    self.bits).to(x.dtype)


def _replace_targets_with_rwkvq(model: nn.Module, sidecar_path: str, rank: int, alpha: float,
                                dropout: float, tmix_targets, quantize_cmix: bool,
                                quantize_head: bool, layers, native=True, device=None) -> list:
    """Swap tmix projections (wrapped in LoRALinear), cmix key/value and the
    head for the sb6 base, by the official .rwkvq key names
    (add_rwkvq.py:40-79)."""
    if native == "hybrid":
        backend = RwkvqHybridLinear
    else:
        backend = RwkvqNativeLinear if native else RwkvqLinear
    n_layer = len(model.blocks)
    sel = set(range(n_layer)) if layers is None else {i % n_layer for i in layers}
    wrapped = []
    for li, blk in enumerate(model.blocks):
        if li not in sel:
            continue
        for name in tmix_targets:
            if getattr(blk.tmix, name, None) is None:
                continue
            base = backend.from_sidecar(sidecar_path, f"blocks.{li}.att.{_TMIX_KEY[name]}.weight",
                                        device)
            setattr(blk.tmix, name, LoRALinear(rank=rank, alpha=alpha, dropout=dropout,
                                               base_module=base))
            wrapped.append(f"tmix.{name}")
        if quantize_cmix:
            for name in ("key", "value"):
                setattr(blk.cmix, name,
                        backend.from_sidecar(sidecar_path, f"blocks.{li}.ffn.{name}.weight", device))
    if quantize_head:
        model.head = backend.from_sidecar(sidecar_path, "head.weight", device)
    return wrapped


def add_lora_rwkvq(model: nn.Module, sidecar_path: str, rank: int = 16, alpha: float = 32.0,
                   dropout: float = 0.0, tmix_targets=TMIX_TARGETS, quantize_cmix: bool = True,
                   quantize_head: bool = True, layers=None, native=True, device=None):
    """QLoRA on the sb6 base of an already loaded model (add_rwkvq.py:82-102):
    returns (model, info) with only the LoRA adapters trainable."""
    wrapped = _replace_targets_with_rwkvq(model, sidecar_path, rank, alpha, dropout, tmix_targets,
                                          quantize_cmix, quantize_head, layers, native, device)
    for p in model.parameters():
        p.requires_grad_(False)
    _unfreeze_adapters(model)
    info = _param_stats(model)
    info["wrapped_per_block"] = sorted(set(wrapped))
    info["num_lora_adapters"] = len(wrapped)
    info["quantize_cmix"] = quantize_cmix
    info["quantize_head"] = quantize_head
    return model, info

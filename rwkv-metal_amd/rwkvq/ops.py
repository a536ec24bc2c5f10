"""torch custom ops over the C ABI: the MLX quantization op surface.

    quantize(w, group_size=64, bits=4)                    <- mx.quantize
    dequantize(w_q, scales, biases, group_size, bits)     <- mx.dequantize
    quantized_matmul(x, w_q, scales, biases, transpose,   <- mx.quantized_matmul
                     group_size, bits)
    pack_codes(codes, bits) / unpack_codes(w_q, bits)     <- the MLX bitstream rule
    quantized_embedding(idx, w_q, scales, biases, ...)    <- nn.QuantizedEmbedding lookup
    quantized_matmul_lora(x, w_q, s, b, z, lora, scale)   <- LoRALinear over a quantized base

Reference call sites: rwkv_metal/lora/finetune.py:88-89 (nn.quantize),
rwkv_metal/lora/lora.py:45-46 (QuantizedLinear.from_linear),
rwkv_metal/lora/rwkvq_native.py:120-122 (quantized_matmul, transpose=True),
tests/dev_pack_native_mlx.py:70 (dequantize), rwkv_metal/lora/rwkvq_native.py:81-90
(packing).  MLX semantics kept: the grouped axis is the last one, leading
dimensions of x fold into M, x and scales are promoted to a common dtype
(equal dtypes stay, any other mix computes in float32), and the gradient of
quantized_matmul flows to x only, as dY through the opposite transpose.

Packed weights are int32 tensors holding the uint32 words bit for bit
(uint32 tensors are accepted and viewed as int32).  Tensors must live on the
ROCm GPU; there is no CPU path.
"""
from __future__ import annotations

import collections
import ctypes
from typing import List, Sequence, Tuple

import torch
from torch import Tensor

from . import _lib
from ._lib import DTYPE_CODE, RQ_EUNSUPPORTED, RqGroupedPlan, RqProblem, check, lib

VALID_BITS = (2, 3, 4, 5, 6, 8)
VALID_GROUP_SIZES = (32, 64, 128)


def _promote(a: torch.dtype, b: torch.dtype) -> torch.dtype:
    return a if a == b else torch.float32


def _check_args(group_size: int, bits: int) -> None:
    if bits not in VALID_BITS:
        raise ValueError(f"bits must be one of {VALID_BITS} (got {bits})")
    if group_size not in VALID_GROUP_SIZES:
        raise ValueError(f"group_size must be one of {VALID_GROUP_SIZES} (got {group_size})")


def _on_gpu(*ts: Tensor) -> None:
    """Every operand on the same GPU: the kernels take raw pointers and run on
    the first operand's device."""
    for t in ts:
        if t.device.type != "cuda":
            raise RuntimeError(
                "rwkvq ops run only on a ROCm GPU (HIP library); got a tensor on "
                f"'{t.device}'. There is no CPU implementation.")
        if t.device != ts[0].device:
            raise ValueError(f"rwkvq ops take every operand on one device; got '{ts[0].device}' "
                             f"and '{t.device}'")


def _float(t: Tensor, name: str) -> None:
    if t.dtype not in DTYPE_CODE:
        raise ValueError(f"{name} must be bfloat16, float16 or float32 (got {t.dtype})")


def _ready(t: Tensor) -> Tensor:
    """Contiguous and 16-byte aligned (the ABI's requirement)."""
    t = t.contiguous()
    if t.numel() and t.data_ptr() % 16:
        t = t.clone()
    return t


def _words(w_q: Tensor) -> Tensor:
    if w_q.dtype == torch.uint32:
        w_q = w_q.view(torch.int32)
    if w_q.dtype != torch.int32:
        raise ValueError(f"packed weights must be int32/uint32 words (got {w_q.dtype})")
    return w_q


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream_on(device: torch.device) -> int:
    """Raw handle of the current stream on `device`.  Read without building a
    torch.cuda.Stream object: that lookup cost more host time than a small
    decode kernel runs on the GPU."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if _raw_stream is not None:
        return _raw_stream(idx)
    return torch.cuda.current_stream(idx).cuda_stream


def _stream(t: Tensor) -> int:
    return _stream_on(t.device)


class _DeviceGuard:
    """torch.cuda.device(idx) that switches only when idx is not current
    (the common case costs one device query)."""
    __slots__ = ("idx", "prev")

    def __init__(self, device: torch.device):
        self.idx = device.index if device.index is not None else torch.cuda.current_device()
        self.prev = -1

    def __enter__(self):
        cur = torch.cuda.current_device()
        if cur != self.idx:
            self.prev = cur
            torch.cuda.set_device(self.idx)
        return self

    def __exit__(self, *exc):
        if self.prev >= 0:
            torch.cuda.set_device(self.prev)
            self.prev = -1
        return False


def _ptr(t: Tensor) -> int:
    return t.data_ptr() if t.numel() else 0


_dispatch_modes = torch._C._len_torch_dispatch_stack
_function_modes = torch._C._len_torch_function_stack
_functorch_active = torch._C._are_functorch_transforms_active


def _direct(*ts: Tensor) -> bool:
    """True when a call may run an op's body without the torch.library
    dispatcher: plain GPU tensors, no autograd to record, no tracing, no
    dispatch or function mode and no functorch transform.  Such a call does
    exactly what the registered op would do and skips about 13 us of host
    dispatch, which is longer than the small launches take on the GPU.
    Anything else (torch.compile, meta and fake tensors, autograd, CPU
    tensors, which the op refuses) goes through the registered op."""
    if _dispatch_modes() or _function_modes() or _functorch_active():
        return False
    grad = torch.is_grad_enabled()
    for t in ts:
        if type(t) is not Tensor or not t.is_cuda or (grad and t.requires_grad):
            return False
    return not torch.compiler.is_compiling()


# --------------------------------------------------------------- quantize

def _quantize_impl(w: Tensor, group_size: int, bits: int) -> Tuple[Tensor, Tensor, Tensor]:
    _on_gpu(w)
    w = _ready(w)
    K = w.shape[-1]
    R = w.numel() // K if K else 0
    lead = w.shape[:-1]
    wq = torch.empty(*lead, K * bits // 32, dtype=torch.int32, device=w.device)
    s = torch.empty(*lead, K // group_size, dtype=w.dtype, device=w.device)
    b = torch.empty_like(s)
    with _DeviceGuard(w.device):
        rc = lib().rq_quantize(_ptr(w), DTYPE_CODE[w.dtype], R, K, group_size, bits, _ptr(wq),
                               _ptr(s), _ptr(b), _stream(w))
    check(rc, "quantize")
    return wq, s, b


_quantize_op = torch.library.custom_op("rwkvq::quantize", _quantize_impl, mutates_args=())


@_quantize_op.register_fake
def _(w, group_size, bits):
    K = w.shape[-1]
    lead = w.shape[:-1]
    return (w.new_empty(*lead, K * bits // 32, dtype=torch.int32),
            w.new_empty(*lead, K // group_size), w.new_empty(*lead, K // group_size))


def quantize(w: Tensor, group_size: int = 64, bits: int = 4) -> Tuple[Tensor, Tensor, Tensor]:
    """mx.quantize (affine): w[..., K] -> (w_q int32[..., K*bits/32], scales, biases)."""
    _check_args(group_size, bits)
    _float(w, "w")
    if w.dim() < 2:
        raise ValueError("quantize expects a matrix (at least 2 dimensions)")
    if w.shape[-1] % group_size:
        raise ValueError(f"the last dimension ({w.shape[-1]}) must be divisible by "
                         f"group_size {group_size}")
    if _direct(w):
        return _quantize_impl(w, group_size, bits)
    return _quantize_op(w, group_size, bits)


# ------------------------------------------------------------- dequantize

def _dequantize_impl(w_q: Tensor, scales: Tensor, biases: Tensor, group_size: int,
                   bits: int) -> Tensor:
    _on_gpu(w_q, scales, biases)
    w_q, scales, biases = _ready(w_q), _ready(scales), _ready(biases.to(scales.dtype))
    K = w_q.shape[-1] * 32 // bits
    R = w_q.numel() // w_q.shape[-1] if w_q.shape[-1] else 0
    out = torch.empty(*w_q.shape[:-1], K, dtype=scales.dtype, device=w_q.device)
    with _DeviceGuard(w_q.device):
        rc = lib().rq_dequantize(_ptr(w_q), _ptr(scales), _ptr(biases), DTYPE_CODE[scales.dtype],
                                 R, K, group_size, bits, _ptr(out), DTYPE_CODE[out.dtype],
                                 _stream(w_q))
    check(rc, "dequantize")
    return out


_dequantize_op = torch.library.custom_op("rwkvq::dequantize", _dequantize_impl,
                                         mutates_args=())


@_dequantize_op.register_fake
def _(w_q, scales, biases, group_size, bits):
    K = w_q.shape[-1] * 32 // bits
    return scales.new_empty(*w_q.shape[:-1], K)


def _check_packed(w_q: Tensor, scales: Tensor, biases: Tensor, group_size: int, bits: int):
    if (w_q.shape[-1] * 32) % bits:
        raise ValueError("packed width is not a whole number of codes")
    K = w_q.shape[-1] * 32 // bits
    if K % group_size:
        raise ValueError(f"unpacked width {K} is not divisible by group_size {group_size}")
    want = (*w_q.shape[:-1], K // group_size)
    if tuple(scales.shape) != want or tuple(biases.shape) != want:
        raise ValueError(f"scales/biases must have shape {want} "
                         f"(got {tuple(scales.shape)} / {tuple(biases.shape)})")
    return K


def dequantize(w_q: Tensor, scales: Tensor, biases: Tensor, group_size: int = 64,
               bits: int = 4) -> Tensor:
    """mx.dequantize: scales*code + biases, evaluated in the scales dtype."""
    _check_args(group_size, bits)
    w_q = _words(w_q)
    _float(scales, "scales")
    _check_packed(w_q, scales, biases, group_size, bits)
    if _direct(w_q, scales, biases):
        return _dequantize_impl(w_q, scales, biases, group_size, bits)
    return _dequantize_op(w_q, scales, biases, group_size, bits)


# ------------------------------------------------------------ embedding

def _embedding_impl(idx: Tensor, w_q: Tensor, scales: Tensor, biases: Tensor, group_size: int,
                  bits: int) -> Tensor:
    _on_gpu(idx, w_q, scales, biases)
    flat = _ready(idx.reshape(-1).to(torch.int64))
    w_q, scales, biases = _ready(w_q), _ready(scales), _ready(biases.to(scales.dtype))
    R, K = w_q.shape[0], w_q.shape[1] * 32 // bits
    out = torch.empty(*idx.shape, K, dtype=scales.dtype, device=w_q.device)
    if out.numel() == 0:
        return out
    with _DeviceGuard(w_q.device):
        rc = lib().rq_embedding(_ptr(flat), flat.numel(), _ptr(w_q), _ptr(scales), _ptr(biases),
                                DTYPE_CODE[scales.dtype], R, K, group_size, bits, _ptr(out),
                                DTYPE_CODE[out.dtype], _stream(w_q))
    check(rc, "quantized_embedding")
    return out


_embedding_op = torch.library.custom_op("rwkvq::quantized_embedding", _embedding_impl,
                                        mutates_args=())


@_embedding_op.register_fake
def _(idx, w_q, scales, biases, group_size, bits):
    return scales.new_empty(*idx.shape, w_q.shape[1] * 32 // bits)


def quantized_embedding(idx: Tensor, w_q: Tensor, scales: Tensor, biases: Tensor,
                        group_size: int = 64, bits: int = 4) -> Tensor:
    """nn.QuantizedEmbedding's lookup: dequantize(table rows idx) in one fused
    gather-dequantize launch; out[..., :] has idx's shape plus the row width,
    in the scales dtype.  Indices outside the table give rows of NaN."""
    _check_args(group_size, bits)
    w_q = _words(w_q)
    _float(scales, "scales")
    if w_q.dim() != 2:
        raise ValueError("quantized_embedding expects a 2-D packed table")
    _check_packed(w_q, scales, biases, group_size, bits)
    if idx.dtype not in (torch.int64, torch.int32, torch.int16, torch.uint8):
        raise ValueError(f"indices must be an integer tensor (got {idx.dtype})")
    if _direct(idx, w_q, scales, biases):
        return _embedding_impl(idx, w_q, scales, biases, group_size, bits)
    return _embedding_op(idx, w_q, scales, biases, group_size, bits)


# ------------------------------------------------------- quantized_matmul

def _qmm_impl(x: Tensor, w_q: Tensor, scales: Tensor, biases: Tensor, transpose: bool,
            group_size: int, bits: int) -> Tensor:
    _on_gpu(x, w_q, scales, biases)
    x, w_q, scales = _ready(x), _ready(w_q), _ready(scales)
    biases = _ready(biases.to(scales.dtype))
    R = w_q.shape[0]
    K = w_q.shape[1] * 32 // bits
    n_out = R if transpose else K
    out_dtype = _promote(x.dtype, scales.dtype)
    m = x.numel() // x.shape[-1] if x.shape[-1] else 0
    y = torch.empty(*x.shape[:-1], n_out, dtype=out_dtype, device=x.device)
    if y.numel() == 0:
        return y
    L = lib()
    with _DeviceGuard(x.device):
        stream = _stream(x)
        # prefill batches with few output tiles over a long contraction split it
        # (rq_qmm_splitk, a per-stream workspace); everything else is rq_qmm
        nbytes = L.rq_qmm_splitk_workspace_bytes(m, R, K, group_size, bits) if (
            transpose and m >= 256) else 0
        if nbytes > 0:
            ws = _splitk_workspace(x.device, stream, nbytes)
            rc = L.rq_qmm_splitk(_ptr(x), DTYPE_CODE[x.dtype], _ptr(w_q), _ptr(scales),
                                 _ptr(biases), DTYPE_CODE[scales.dtype], m, R, K, group_size,
                                 bits, _ptr(y), DTYPE_CODE[out_dtype], ws.data_ptr(), ws.numel(),
                                 stream)
        else:
            rc = L.rq_qmm(_ptr(x), DTYPE_CODE[x.dtype], _ptr(w_q), _ptr(scales), _ptr(biases),
                          DTYPE_CODE[scales.dtype], m, R, K, group_size, bits,
                          1 if transpose else 0, _ptr(y), DTYPE_CODE[out_dtype], stream)
    check(rc, "quantized_matmul")
    return y


_splitk_workspaces: "collections.OrderedDict" = collections.OrderedDict()


def _splitk_workspace(device: torch.device, stream: int, nbytes: int) -> Tensor:
    """The split-K GEMM's partial tiles, one buffer per (device, stream) and at
    most _GRAD_WORKSPACES_MAX of them (least recently used out), as for the
    gradient workspaces; it needs no initialisation.  Allocated while its
    stream is current, so torch's caching allocator reuses a dropped one only
    on that stream, after the work queued there."""
    key = (device.index, stream)
    ws = _splitk_workspaces.pop(key, None)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
    _splitk_workspaces[key] = ws
    while len(_splitk_workspaces) > _GRAD_WORKSPACES_MAX:
        _splitk_workspaces.popitem(last=False)
    return ws


_qmm_op = torch.library.custom_op("rwkvq::quantized_matmul", _qmm_impl,
                                  mutates_args=())


@_qmm_op.register_fake
def _(x, w_q, scales, biases, transpose, group_size, bits):
    R = w_q.shape[0]
    K = w_q.shape[1] * 32 // bits
    return x.new_empty(*x.shape[:-1], R if transpose else K,
                       dtype=_promote(x.dtype, scales.dtype))


def _qmm_setup(ctx, inputs, output):
    x, w_q, scales, biases, transpose, group_size, bits = inputs
    ctx.save_for_backward(w_q, scales, biases)
    ctx.transpose, ctx.group_size, ctx.bits = transpose, group_size, bits
    ctx.x_dtype = x.dtype


def _qmm_backward(ctx, grad):
    w_q, scales, biases = ctx.saved_tensors
    dx = None
    if ctx.needs_input_grad[0]:
        dx = _qmm_op(grad.contiguous(), w_q, scales, biases, not ctx.transpose, ctx.group_size,
                     ctx.bits).to(ctx.x_dtype)
    return dx, None, None, None, None, None, None


_qmm_op.register_autograd(_qmm_backward, setup_context=_qmm_setup)


def quantized_matmul(x: Tensor, w_q: Tensor, scales: Tensor, biases: Tensor,
                     transpose: bool = True, group_size: int = 64, bits: int = 4) -> Tensor:
    """mx.quantized_matmul.  transpose=True: x @ W^T ; transpose=False: x @ W."""
    _check_args(group_size, bits)
    w_q = _words(w_q)
    _float(x, "x")
    _float(scales, "scales")
    if w_q.dim() != 2:
        raise ValueError("quantized_matmul expects a 2-D packed weight")
    K = _check_packed(w_q, scales, biases, group_size, bits)
    n_in = K if transpose else w_q.shape[0]
    if x.shape[-1] != n_in:
        raise ValueError(f"x has inner dimension {x.shape[-1]} but the quantized weight expects "
                         f"{n_in} (transpose={transpose})")
    if _direct(x, w_q, scales, biases):
        return _qmm_impl(x, w_q, scales, biases, bool(transpose), group_size, bits)
    return _qmm_op(x, w_q, scales, biases, bool(transpose), group_size, bits)


def lora_down(x: Tensor, a: Tensor) -> Tensor:
    """x @ a^T for the QLoRA layer's low-rank products (rank = a.shape[0]):
    z = x A^T in the forward, u = dY B (a = B^T) in the backward
    (rwkv_metal/lora/lora.py:58-63).  bf16 CUDA operands with a rank of 16,
    32, 48 or 64 and an inner size that is a multiple of 32 run rq_lora_down
    (one HIP launch); other operands take torch's matmul, fp32 x against a
    bf16 adapter in fp32 with z rounded once to bf16 (the form the fused
    kernels produce)."""
    if x.shape[-1] != a.shape[-1]:
        raise ValueError(f"lora_down: x has inner size {x.shape[-1]}, a has {a.shape[-1]}")
    rank, k = a.shape[0], a.shape[-1]
    if not (x.is_cuda and x.dtype == a.dtype == torch.bfloat16 and rank in (16, 32, 48, 64)
            and k % 32 == 0 and k > 0):
        if x.dtype == torch.float32 and a.dtype == torch.bfloat16:
            return (x @ a.float().t()).to(torch.bfloat16)
        return x @ a.t()
    _on_gpu(x, a)
    x2 = _ready(x.reshape(-1, k))
    a = _ready(a)
    z = torch.empty(x2.shape[0], rank, dtype=torch.bfloat16, device=x.device)
    if x2.shape[0]:
        with _DeviceGuard(x.device):
            rc = lib().rq_lora_down(_ptr(x2), x2.shape[0], k, _ptr(a), rank, _ptr(z),
                                    _stream_on(x.device))
        if rc:
            check(rc, "lora_down")
    return z.reshape(*x.shape[:-1], rank)


_grad_workspaces: "collections.OrderedDict" = collections.OrderedDict()
_GRAD_WORKSPACES_MAX = 8


def _lora_workspace(device: torch.device, stream: int, nbytes: int) -> Tensor:
    """A zero-filled workspace for rq_lora_grads, one per (device, stream):
    every call leaves it zeroed for the next, and calls on one stream run in
    order, so they can share it.  At most _GRAD_WORKSPACES_MAX are kept, least
    recently used first out.  Each is allocated while its stream is current,
    so torch's caching allocator hands a dropped one only to later
    allocations on that same stream, after the work queued there."""
    key = (device.index, stream)
    ws = _grad_workspaces.pop(key, None)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=device)
    _grad_workspaces[key] = ws
    while len(_grad_workspaces) > _GRAD_WORKSPACES_MAX:
        _grad_workspaces.popitem(last=False)
    return ws


_grad_ws_bytes: dict = {}  # (m, k, n, rank, dA?, dB?) -> rq_lora_grads_workspace_bytes


def lora_grads(x: Tensor | None, u: Tensor | None, dy: Tensor | None, z: Tensor | None,
               scale: float) -> Tuple[Tensor | None, Tensor | None]:
    """The QLoRA adapter gradients of rwkv_metal/lora/lora.py:58-63 under
    nn.value_and_grad (finetune.py:141): dA = scale * u^T x [rank, K] and
    dB = scale * dY^T z [N, rank], bf16, in one rq_lora_grads launch
    (rq_lora_grads_f32 when x and dY are fp32, the reference's default
    activations; u and z are bf16 either way).  Pass None for both operands
    of a gradient that is not needed."""
    want_a, want_b = x is not None, dy is not None
    ref = x if want_a else dy
    if ref is None:
        return None, None
    _on_gpu(*[t for t in (x, u, dy, z) if t is not None])
    q = u if want_a else z
    rank = q.shape[-1]
    xdt = ref.dtype
    if not (rank in (16, 32, 48, 64) and xdt in (torch.bfloat16, torch.float32)
            and all(t is None or t.dtype == xdt for t in (x, dy))
            and all(t is None or t.dtype == torch.bfloat16 for t in (u, z))
            and (not want_a or x.shape[-1] % 8 == 0) and (not want_b or dy.shape[-1] % 8 == 0)):
        # ranks and dtypes the launch does not cover: fp32 products on the GPU
        da = (scale * (u.float().t() @ x.float())).to(u.dtype) if want_a else None
        db = (scale * (dy.float().t() @ z.float())).to(z.dtype) if want_b else None
        return da, db
    m = ref.numel() // ref.shape[-1]
    x2 = _ready(x.reshape(m, x.shape[-1])) if want_a else None
    u2 = _ready(u.reshape(m, rank)) if want_a else None
    dy2 = _ready(dy.reshape(m, dy.shape[-1])) if want_b else None
    z2 = _ready(z.reshape(m, rank)) if want_b else None
    K = x2.shape[1] if want_a else 0
    N = dy2.shape[1] if want_b else 0
    da = torch.empty(rank, K, dtype=torch.bfloat16, device=ref.device) if want_a else None
    db = torch.empty(N, rank, dtype=torch.bfloat16, device=ref.device) if want_b else None
    L = lib()
    with _DeviceGuard(ref.device):
        stream = _stream_on(ref.device)
        key = (m, K, N, rank, want_a, want_b)
        nbytes = _grad_ws_bytes.get(key)
        if nbytes is None:
            nbytes = L.rq_lora_grads_workspace_bytes(m, K, N, rank, int(want_a), int(want_b))
            check(nbytes if nbytes < 0 else 0, "lora_grads")
            if len(_grad_ws_bytes) > 4096:
                _grad_ws_bytes.clear()
            _grad_ws_bytes[key] = nbytes
        ws = _lora_workspace(ref.device, stream, int(nbytes)) if nbytes > 0 else None
        fn = L.rq_lora_grads_f32 if xdt == torch.float32 else L.rq_lora_grads
        rc = fn(_ptr(x2) if want_a else 0, _ptr(u2) if want_a else 0,
                _ptr(dy2) if want_b else 0, _ptr(z2) if want_b else 0, m, K, N,
                rank, float(scale), _ptr(da) if want_a else 0,
                _ptr(db) if want_b else 0, ws.data_ptr() if ws is not None else 0,
                ws.numel() if ws is not None else 0, stream)
    check(rc, "lora_grads")
    return da, db


def _qmm_lora_fused(x: Tensor, w_q: Tensor, scales: Tensor, biases: Tensor, z: Tensor,
                    lora: Tensor, scale: float, transpose: bool, group_size: int, bits: int):
    """rq_qmm_lora on 2-D operands; None where the fused kernels do not apply."""
    if not (x.dtype in (torch.bfloat16, torch.float32) and z.dtype == lora.dtype == torch.bfloat16):
        return None
    x, w_q, scales = _ready(x), _ready(w_q), _ready(scales)
    biases, z, lora = _ready(biases.to(scales.dtype)), _ready(z), _ready(lora)
    R, K = w_q.shape[0], w_q.shape[1] * 32 // bits
    m, rank = x.shape[0], z.shape[1]
    y = torch.empty(m, R if transpose else K, dtype=_promote(x.dtype, scales.dtype),
                    device=x.device)
    with _DeviceGuard(x.device):
        rc = lib().rq_qmm_lora(_ptr(x), DTYPE_CODE[x.dtype], _ptr(w_q), _ptr(scales), _ptr(biases),
                               DTYPE_CODE[scales.dtype], m, R, K, group_size, bits,
                               1 if transpose else 0, _ptr(z), _ptr(lora), rank, float(scale),
                               _ptr(y), DTYPE_CODE[y.dtype], _stream(x))
    if rc == RQ_EUNSUPPORTED:
        return None
    check(rc, "quantized_matmul_lora")
    return y


def qlora_fused(x: Tensor, w_q: Tensor, scales: Tensor, biases: Tensor, a: Tensor,
                lora: Tensor, scale: float, transpose: bool = True, group_size: int = 64,
                bits: int = 4, out_dtype: torch.dtype | None = None):
    """The QLoRA layer product in one rq_qlora launch, its down-projection
    inside the GEMM: (y, z) with z = x @ a^T [m, rank] (bf16) and
    y = quantized_matmul(x, ...) + scale * z @ lora^T.  Forward: a = lora_a,
    lora = lora_b; dX: a = lora_b^T, lora = lora_a^T (transpose=False), z is
    then u = dY @ lora_b.  x is 2-D.  y is in out_dtype if given (bf16 or
    fp32), else in MLX's promotion of x and the scales.  None where the fused
    kernels do not apply (see rq_qlora); no autograd (rwkvq.lora
    differentiates the layer)."""
    _check_args(group_size, bits)
    w_q = _words(w_q)
    K = _check_packed(w_q, scales, biases, group_size, bits)
    n_in, n_out = (K, w_q.shape[0]) if transpose else (w_q.shape[0], K)
    rank = a.shape[0]
    if (x.dim() != 2 or x.shape[1] != n_in or tuple(a.shape) != (rank, n_in)
            or tuple(lora.shape) != (n_out, rank)):
        raise ValueError("qlora_fused: x, a and lora shapes do not agree")
    if not (x.dtype in (torch.bfloat16, torch.float32) and a.dtype == lora.dtype == torch.bfloat16
            and rank == 16):
        return None
    _on_gpu(x, w_q, scales, biases, a, lora)
    x, w_q, scales, a, lora = _ready(x), _ready(w_q), _ready(scales), _ready(a), _ready(lora)
    biases = _ready(biases.to(scales.dtype))
    m = x.shape[0]
    y = torch.empty(m, n_out, dtype=out_dtype or _promote(x.dtype, scales.dtype), device=x.device)
    z = torch.empty(m, rank, dtype=torch.bfloat16, device=x.device)
    if m == 0:
        return y, z
    with _DeviceGuard(x.device):
        rc = lib().rq_qlora(_ptr(x), DTYPE_CODE[x.dtype], _ptr(w_q), _ptr(scales), _ptr(biases),
                            DTYPE_CODE[scales.dtype], m, w_q.shape[0], K, group_size, bits,
                            1 if transpose else 0, _ptr(a), _ptr(lora), rank, float(scale),
                            _ptr(z), _ptr(y), DTYPE_CODE[y.dtype], _stream(x))
    if rc == RQ_EUNSUPPORTED:
        return None
    check(rc, "qlora_fused")
    return y, z


def qlora_dx_fused(dy: Tensor, w_q: Tensor, scales: Tensor, biases: Tensor, lora_a: Tensor,
                   lora_b: Tensor, scale: float, group_size: int = 64, bits: int = 4,
                   out_dtype: torch.dtype | None = None):
    """The QLoRA layer's dX in one rq_qlora_dx launch from the adapters as
    the layer stores them (lora_a [rank, K], lora_b [R, rank]): (dx, u) with
    u = dy @ lora_b [m, rank] (bf16) computed inside the transposed GEMM and
    dx = quantized_matmul(dy, ..., transpose=False) + scale * u @ lora_a;
    equal bit for bit to qlora_fused(dy, ..., lora_b^T, lora_a^T, scale,
    False), without the transposed copies.  dy is 2-D.  None where the fused
    kernels do not apply; no autograd."""
    _check_args(group_size, bits)
    w_q = _words(w_q)
    K = _check_packed(w_q, scales, biases, group_size, bits)
    R = w_q.shape[0]
    rank = lora_a.shape[0]
    if (dy.dim() != 2 or dy.shape[1] != R or tuple(lora_a.shape) != (rank, K)
            or tuple(lora_b.shape) != (R, rank)):
        raise ValueError("qlora_dx_fused: dy, lora_a and lora_b shapes do not agree")
    if not (dy.dtype in (torch.bfloat16, torch.float32)
            and lora_a.dtype == lora_b.dtype == torch.bfloat16 and rank == 16):
        return None
    _on_gpu(dy, w_q, scales, biases, lora_a, lora_b)
    dy, w_q, scales = _ready(dy), _ready(w_q), _ready(scales)
    lora_a, lora_b = lora_a.contiguous(), _ready(lora_b)
    biases = _ready(biases.to(scales.dtype))
    m = dy.shape[0]
    dx = torch.empty(m, K, dtype=out_dtype or _promote(dy.dtype, scales.dtype), device=dy.device)
    u = torch.empty(m, rank, dtype=torch.bfloat16, device=dy.device)
    if m == 0:
        return dx, u
    with _DeviceGuard(dy.device):
        rc = lib().rq_qlora_dx(_ptr(dy), DTYPE_CODE[dy.dtype], _ptr(w_q), _ptr(scales),
                               _ptr(biases), DTYPE_CODE[scales.dtype], m, R, K, group_size, bits,
                               _ptr(lora_a), _ptr(lora_b), rank, float(scale), _ptr(u), _ptr(dx),
                               DTYPE_CODE[dx.dtype], _stream(dy))
    if rc == RQ_EUNSUPPORTED:
        return None
    check(rc, "qlora_dx_fused")
    return dx, u


def quantized_matmul_lora(x: Tensor, w_q: Tensor, scales: Tensor, biases: Tensor, z: Tensor,
                          lora: Tensor, scale: float, transpose: bool = True,
                          group_size: int = 64, bits: int = 4) -> Tensor:
    """quantized_matmul(x, ...) + scale * z @ lora^T: the QLoRA layer's low-rank
    term (rwkv_metal/lora/lora.py:58-63; z = x @ lora_a^T, lora = lora_b; for
    dX, z = dY @ lora_b and lora = lora_a^T) added in the GEMM's output stage
    where the 64-wide-stage kernels run (rq_qmm_lora), computed separately
    otherwise.  z [..., rank], lora [n_out, rank].  No autograd here:
    rwkvq.lora.LoRALinear differentiates the layer."""
    _check_args(group_size, bits)
    w_q = _words(w_q)
    K = _check_packed(w_q, scales, biases, group_size, bits)
    n_in, n_out = (K, w_q.shape[0]) if transpose else (w_q.shape[0], K)
    if x.shape[-1] != n_in or z.shape[:-1] != x.shape[:-1] or tuple(lora.shape) != (n_out, z.shape[-1]):
        raise ValueError("quantized_matmul_lora: x, z and lora shapes do not agree")
    _on_gpu(x, w_q, scales, biases, z, lora)
    lead = x.shape[:-1]
    x2, z2 = x.reshape(-1, n_in), z.reshape(-1, z.shape[-1])
    y = None
    if z2.shape[-1] in (16, 32, 48, 64) and x2.shape[0] > 0:
        y = _qmm_lora_fused(x2, w_q, scales, biases, z2, lora, scale, transpose, group_size, bits)
    if y is None:
        y = quantized_matmul(x2, w_q, scales, biases, transpose, group_size, bits)
        ct = _promote(y.dtype, z2.dtype)
        y = (y.to(ct) + scale * (z2.to(ct) @ lora.to(ct).t())).to(y.dtype)
    return y.reshape(*lead, n_out)


class BoundQmm:
    """One validated quantized_matmul (either transpose) with a fixed output
    buffer: run() is a single rq_qmm call (rq_qmm_splitk, with a workspace of
    its own, where the split-K plan applies) on the current stream, with no
    per-call validation, allocation or custom-op dispatch.  For serving or
    training loops that repeat the same product on the same buffers (and for
    timing the kernel rather than the Python dispatch).  Same semantics and
    output dtype as quantized_matmul; x may be overwritten in place between
    runs."""

    def __init__(self, x: Tensor, w_q: Tensor, scales: Tensor, biases: Tensor,
                 transpose: bool = True, group_size: int = 64, bits: int = 4,
                 out: Tensor | None = None):
        _check_args(group_size, bits)
        w_q = _words(w_q)
        _float(x, "x")
        _float(scales, "scales")
        _on_gpu(x, w_q, scales, biases)
        if w_q.dim() != 2:
            raise ValueError("quantized_matmul expects a 2-D packed weight")
        K = _check_packed(w_q, scales, biases, group_size, bits)
        R = w_q.shape[0]
        n_in, n_out = (K, R) if transpose else (R, K)
        if x.shape[-1] != n_in:
            raise ValueError(f"x has inner dimension {x.shape[-1]} but the quantized weight "
                             f"expects {n_in} (transpose={transpose})")
        if not x.is_contiguous():
            raise ValueError("BoundQmm needs a contiguous x (it is read in place on every run)")
        w_q, scales = _ready(w_q), _ready(scales)
        biases = _ready(biases.to(scales.dtype))
        ydt = _promote(x.dtype, scales.dtype)
        y = out if out is not None else torch.empty(*x.shape[:-1], n_out, dtype=ydt,
                                                    device=x.device)
        if y.dtype != ydt or not y.is_contiguous() or tuple(y.shape) != (*x.shape[:-1], n_out):
            raise ValueError(f"BoundQmm: output must be a contiguous {ydt} tensor of shape "
                             f"{(*x.shape[:-1], n_out)}")
        self._keep = (x, w_q, scales, biases)
        self.out, self.device = y, x.device
        m = x.numel() // x.shape[-1] if x.shape[-1] else 0
        self._args = (x.data_ptr(), DTYPE_CODE[x.dtype], w_q.data_ptr(), scales.data_ptr(),
                      biases.data_ptr(), DTYPE_CODE[scales.dtype], m, R, K, group_size, bits,
                      1 if transpose else 0, y.data_ptr(), DTYPE_CODE[ydt])
        self._empty = y.numel() == 0
        self._guard, self._fn = _DeviceGuard(self.device), lib().rq_qmm
        nbytes = lib().rq_qmm_splitk_workspace_bytes(m, R, K, group_size, bits) if (
            transpose and m >= 256) else 0
        if nbytes > 0:   # its own partial-tile workspace, held with the bound buffers
            self.workspace = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
            a = self._args
            self._args = (*a[:11], a[12], a[13], self.workspace.data_ptr(), nbytes)
            self._fn = lib().rq_qmm_splitk

    def run(self) -> Tensor:
        if not self._empty:
            with self._guard:
                rc = self._fn(*self._args, _stream_on(self.device))
            if rc:
                check(rc, "quantized_matmul")
        return self.out


class GroupedQmv:
    """A validated set of independent decode products y_i = x_i @ W_i^T
    (m <= 16): one ctypes call and, where the planned kernel covers the
    problems (rq_grouped_plan_*), one kernel launch per run(); otherwise
    rq_qmm_grouped's launches.  All x_i share m and dtype; all W_i share
    bits, group size and the scales dtype.  The plan keeps references to every
    tensor, so run() may be called repeatedly (e.g. one decode step each)."""

    PLAN_MIN_BLOCKS = 1024  # below this many 64-row blocks the K-split launches are faster

    def __init__(self, xs: Sequence[Tensor], ws: Sequence[Tuple[Tensor, Tensor, Tensor]],
                 group_size: int = 64, bits: int = 4, out: Sequence[Tensor] | None = None,
                 planned: bool | None = None):
        _check_args(group_size, bits)
        if len(xs) != len(ws):
            raise ValueError("need one weight triple per activation")
        if not xs:
            raise ValueError("grouped_qmv needs at least one problem")
        x0 = xs[0]
        _on_gpu(x0)
        m = x0.numel() // x0.shape[-1]
        if not 1 <= m <= 16:
            raise ValueError(f"grouped_qmv: m must be in [1, 16] (got {m})")
        sdt = ws[0][1].dtype
        ydt = _promote(x0.dtype, sdt)
        self.probs = (RqProblem * len(xs))()
        self._keep, self.outs = [], []
        for i, (x, (w_q, s, b)) in enumerate(zip(xs, ws)):
            _on_gpu(x0, x, w_q, s, b)
            w_q = _words(w_q)
            K = _check_packed(w_q, s, b, group_size, bits)
            if x.dtype != x0.dtype or s.dtype != sdt or x.numel() // x.shape[-1] != m:
                raise ValueError("grouped_qmv: every problem must share m and dtypes")
            if x.shape[-1] != K:
                raise ValueError(f"grouped_qmv: problem {i}: x width {x.shape[-1]} != {K}")
            x, w_q, s, b = _ready(x), _ready(w_q), _ready(s), _ready(b.to(sdt))
            y = out[i] if out is not None else torch.empty(
                *x.shape[:-1], w_q.shape[0], dtype=ydt, device=x.device)
            if y.dtype != ydt or not y.is_contiguous() or y.shape[-1] != w_q.shape[0]:
                raise ValueError(f"grouped_qmv: bad output buffer for problem {i}")
            self._keep += [x, w_q, s, b]
            self.outs.append(y)
            self.probs[i] = RqProblem(x.data_ptr(), w_q.data_ptr(), s.data_ptr(), b.data_ptr(),
                                      y.data_ptr(), w_q.shape[0], K)
        self.n, self.m, self.device = len(xs), m, x0.device
        self.codes = (DTYPE_CODE[x0.dtype], DTYPE_CODE[sdt], DTYPE_CODE[ydt])
        self.group_size, self.bits = group_size, bits
        # A device-side schedule (one launch per run) where the planned kernel
        # covers every problem and the set is large enough (planned=None), or
        # always (True: an uncovered set raises) or never (False).
        self.plan, self._table = None, None
        blocks = sum((w[0].shape[0] + 63) // 64 for w in ws)
        if planned is False or (planned is None and blocks < self.PLAN_MIN_BLOCKS):
            return
        L = lib()
        nbytes = L.rq_grouped_plan_table_bytes(self.probs, self.n)
        check(nbytes if nbytes < 0 else 0, "grouped_qmv plan")
        table = torch.empty(max(int(nbytes), 16), dtype=torch.uint8, device=self.device)
        plan = RqGroupedPlan()
        with _DeviceGuard(self.device):
            rc = L.rq_grouped_plan_init(self.probs, self.n, *self.codes, self.m, group_size, bits,
                                        table.data_ptr(), table.numel(), ctypes.byref(plan),
                                        _stream_on(self.device))
        if rc == RQ_EUNSUPPORTED and not planned:
            return
        check(rc, "grouped_qmv plan")
        self.plan, self._table = plan, table
        self._plan_ref = ctypes.byref(self.plan)

    def run(self) -> List[Tensor]:
        with _DeviceGuard(self.device):
            stream = _stream_on(self.device)
            if self.plan is not None:
                rc = lib().rq_grouped_plan_run(self._plan_ref, stream)
            else:
                rc = lib().rq_qmm_grouped(self.probs, self.n, *self.codes, self.m,
                                          self.group_size, self.bits, stream)
        if rc:
            check(rc, "grouped_qmv")
        return self.outs


def grouped_qmv(xs: Sequence[Tensor], ws: Sequence[Tuple[Tensor, Tensor, Tensor]],
                group_size: int = 64, bits: int = 4, out: Sequence[Tensor] | None = None
                ) -> List[Tensor]:
    """One-shot form of GroupedQmv: y_i = x_i @ W_i^T for every i."""
    if not xs:
        return []
    return GroupedQmv(xs, ws, group_size, bits, out).run()


# ---------------------------------------------------------- pack / unpack

def _pack_impl(codes: Tensor, bits: int) -> Tensor:
    _on_gpu(codes)
    codes = _ready(codes)
    K = codes.shape[-1]
    R = codes.numel() // K if K else 0
    wq = torch.empty(*codes.shape[:-1], K * bits // 32, dtype=torch.int32, device=codes.device)
    with _DeviceGuard(codes.device):
        rc = lib().rq_pack(_ptr(codes), R, K, bits, _ptr(wq), _stream(codes))
    check(rc, "pack_codes")
    return wq


_pack_op = torch.library.custom_op("rwkvq::pack_codes", _pack_impl, mutates_args=())


@_pack_op.register_fake
def _(codes, bits):
    return codes.new_empty(*codes.shape[:-1], codes.shape[-1] * bits // 32, dtype=torch.int32)


def _unpack_impl(w_q: Tensor, bits: int) -> Tensor:
    _on_gpu(w_q)
    w_q = _ready(w_q)
    K = w_q.shape[-1] * 32 // bits
    R = w_q.numel() // w_q.shape[-1] if w_q.shape[-1] else 0
    codes = torch.empty(*w_q.shape[:-1], K, dtype=torch.uint8, device=w_q.device)
    with _DeviceGuard(w_q.device):
        rc = lib().rq_unpack(_ptr(w_q), R, K, bits, _ptr(codes), _stream(w_q))
    check(rc, "unpack_codes")
    return codes


_unpack_op = torch.library.custom_op("rwkvq::unpack_codes", _unpack_impl, mutates_args=())


@_unpack_op.register_fake
def _(w_q, bits):
    return w_q.new_empty(*w_q.shape[:-1], w_q.shape[-1] * 32 // bits, dtype=torch.uint8)


def pack_codes(codes: Tensor, bits: int) -> Tensor:
    """codes uint8[..., K] (K % 32 == 0) -> MLX bitstream words int32[..., K*bits/32]."""
    if bits not in VALID_BITS:
        raise ValueError(f"bits must be one of {VALID_BITS} (got {bits})")
    if codes.dtype != torch.uint8:
        raise ValueError("codes must be uint8")
    if codes.shape[-1] % 32:
        raise ValueError("the code row length must be a multiple of 32")
    if _direct(codes):
        return _pack_impl(codes, bits)
    return _pack_op(codes, bits)


def unpack_codes(w_q: Tensor, bits: int) -> Tensor:
    """Inverse of pack_codes."""
    if bits not in VALID_BITS:
        raise ValueError(f"bits must be one of {VALID_BITS} (got {bits})")
    w_q = _words(w_q)
    if w_q.shape[-1] % bits:
        raise ValueError("packed width must be a multiple of bits words")
    if _direct(w_q):
        return _unpack_impl(w_q, bits)
    return _unpack_op(w_q, bits)

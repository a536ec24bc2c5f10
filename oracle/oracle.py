"""ctypes wrapper over oracle/rq_oracle.c -- TEST INFRASTRUCTURE ONLY.

The CPU restatement of rwkv-metal's group-affine quantized-linear path (MLX
affine quantize / pack / dequantize / quantized_matmul, see rq_oracle.c for the
reference citations).  Imported only by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker, never as the product.

All functions take and return CPU torch tensors.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "librq_oracle.so")

DT = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}

_lib = None


def build() -> str:
    """Compile the oracle with gcc (oracle/Makefile)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"oracle library not built: {_LIB_PATH} (run make -C oracle)")
        L = ctypes.CDLL(_LIB_PATH)
        i64, i32, vp = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p
        L.rqo_quantize.argtypes = [vp, i32, i64, i64, i32, i32, vp, vp, vp]
        L.rqo_pack.argtypes = [vp, i64, i64, i32, vp]
        L.rqo_unpack.argtypes = [vp, i64, i64, i32, vp]
        L.rqo_dequantize.argtypes = [vp, vp, vp, i32, i64, i64, i32, i32, vp, i32]
        L.rqo_qmm.argtypes = [vp, i32, vp, vp, vp, i32, i64, i64, i64, i32, i32, i32, vp, i32, i32,
                              i32]
        L.rqo_qmv_bf16.argtypes = [vp, vp, vp, vp, i64, i64, i64, i32, i32, vp, i32]
        L.rqo_count_ties.argtypes = [vp, i32, i64, i64, i32, i32]
        L.rqo_count_ties.restype = i64
        L.rqo_round_bf16.argtypes = [ctypes.c_float]
        L.rqo_round_bf16.restype = ctypes.c_float
        L.rqo_max_threads.restype = i32
        L.rqo_sb6_codes.argtypes = [vp, i64, i64, i32, vp]
        L.rqo_sb6_scale_min.argtypes = [vp, vp, i64, i64, i32, i32, vp, vp]
        L.rqo_sb6_dequantize.argtypes = [vp, vp, vp, i64, i64, i32, i32, vp]
        _lib = L
    return _lib


def _p(t: torch.Tensor) -> int:
    assert t.device.type == "cpu" and t.is_contiguous()
    return t.data_ptr()


def promote(a: torch.dtype, b: torch.dtype) -> torch.dtype:
    return a if a == b else torch.float32


def quantize(w: torch.Tensor, group_size: int = 64, bits: int = 4):
    """(w_q uint32-as-int32 [R, K*bits/32], scales [R, K/gs], biases [R, K/gs]) in w.dtype."""
    w = w.contiguous()
    R, K = w.shape
    wq = torch.zeros(R, K * bits // 32, dtype=torch.int32)
    s = torch.empty(R, K // group_size, dtype=w.dtype)
    b = torch.empty(R, K // group_size, dtype=w.dtype)
    rc = lib().rqo_quantize(_p(w), DT[w.dtype], R, K, group_size, bits, _p(wq), _p(s), _p(b))
    if rc != 0:
        raise ValueError(f"oracle quantize rejected arguments (rc={rc})")
    return wq, s, b


def count_ties(w: torch.Tensor, group_size: int = 64, bits: int = 4) -> int:
    """Exact half-integer quotients that quantize() rounds on w (each group's
    q0 and every code before clipping): where rint and round-half-away differ."""
    w = w.contiguous()
    R, K = w.shape
    n = lib().rqo_count_ties(_p(w), DT[w.dtype], R, K, group_size, bits)
    if n < 0:
        raise ValueError("oracle count_ties rejected arguments")
    return int(n)


def pack(codes: torch.Tensor, bits: int) -> torch.Tensor:
    codes = codes.to(torch.uint8).contiguous()
    R, K = codes.shape
    wq = torch.zeros(R, K * bits // 32, dtype=torch.int32)
    lib().rqo_pack(_p(codes), R, K, bits, _p(wq))
    return wq


def unpack(wq: torch.Tensor, bits: int) -> torch.Tensor:
    wq = wq.contiguous()
    R, W = wq.shape
    K = W * 32 // bits
    codes = torch.empty(R, K, dtype=torch.uint8)
    lib().rqo_unpack(_p(wq), R, K, bits, _p(codes))
    return codes


def dequantize(wq, scales, biases, group_size=64, bits=4, out_dtype=None):
    wq, scales, biases = wq.contiguous(), scales.contiguous(), biases.contiguous()
    R, W = wq.shape
    K = W * 32 // bits
    out_dtype = out_dtype or scales.dtype
    out = torch.empty(R, K, dtype=out_dtype)
    rc = lib().rqo_dequantize(_p(wq), _p(scales), _p(biases), DT[scales.dtype], R, K,
                              group_size, bits, _p(out), DT[out_dtype])
    if rc != 0:
        raise ValueError(f"oracle dequantize rejected arguments (rc={rc})")
    return out


def quantized_matmul(x, wq, scales, biases, transpose=True, group_size=64, bits=4,
                     out_dtype=None, nthreads=0, weights="mlx"):
    """weights="mlx": the weights are dequantize()'s values (each of s*q and
    +b rounded to the promoted dtype, as MLX's tiled qmm dequantizes);
    weights="exact": s*q + b in double, unrounded (what MLX's qmv computes by
    applying s and b to per-group sums).  For N(0, 0.02) weights the two
    differ by up to ~1% relative: the bias is several times the weight, so
    rounding s*q to bf16 costs more than rounding w."""
    if weights not in ("mlx", "exact"):
        raise ValueError("weights must be 'mlx' or 'exact'")
    x, wq, scales, biases = x.contiguous(), wq.contiguous(), scales.contiguous(), biases.contiguous()
    R, W = wq.shape
    K = W * 32 // bits
    lead = x.shape[:-1]
    m = 1
    for d in lead:
        m *= d
    out_dtype = out_dtype or promote(x.dtype, scales.dtype)
    n_out = R if transpose else K
    if x.shape[-1] != (K if transpose else R):
        raise ValueError("x inner dimension does not match the packed weight")
    y = torch.empty(*lead, n_out, dtype=out_dtype)
    rc = lib().rqo_qmm(_p(x), DT[x.dtype], _p(wq), _p(scales), _p(biases), DT[scales.dtype], m,
                       R, K, group_size, bits, 1 if transpose else 0, _p(y), DT[out_dtype],
                       nthreads, 1 if weights == "exact" else 0)
    if rc != 0:
        raise ValueError(f"oracle qmm rejected arguments (rc={rc})")
    return y


def qmv_bf16(x, wq, scales, biases, group_size=64, bits=4, nthreads=0):
    """Timed CPU baseline form of the GEMV (bf16 in / bf16 out)."""
    R, W = wq.shape
    K = W * 32 // bits
    m = x.numel() // K
    y = torch.empty(m, R, dtype=torch.bfloat16)
    rc = lib().rqo_qmv_bf16(_p(x), _p(wq), _p(scales), _p(biases), m, R, K, group_size, bits,
                            _p(y), nthreads)
    if rc != 0:
        raise ValueError(f"oracle qmv rejected arguments (rc={rc})")
    return y


def max_threads() -> int:
    return int(lib().rqo_max_threads())


# ----------------------------------------------------------- sb6 / K3

def sb6_codes(qblk: torch.Tensor, rows: int, cols: int, xbits: int) -> torch.Tensor:
    """Codes uint8[rows, cols] of a K3-interleaved sb6 tensor."""
    qblk = qblk.contiguous()
    codes = torch.empty(rows, cols, dtype=torch.uint8)
    lib().rqo_sb6_codes(_p(qblk), rows, cols, xbits, _p(codes))
    return codes


def sb6_scale_min(qsqm, ddm, rows, cols, gw_sb, clamp=False):
    """(scale, min) fp32 [rows, cols/32]: f16(qs*d), f16(qm*dm); clamp applies
    max(scale, 1e-8) as the native repack does."""
    qsqm, ddm = qsqm.contiguous(), ddm.contiguous()
    sc = torch.empty(rows, cols // 32, dtype=torch.float32)
    mn = torch.empty_like(sc)
    lib().rqo_sb6_scale_min(_p(qsqm), _p(ddm.view(torch.int16)), rows, cols, gw_sb,
                            1 if clamp else 0, _p(sc), _p(mn))
    return sc, mn


def sb6_dequantize(qblk, qsqm, ddm, rows, cols, gw_sb, xbits) -> torch.Tensor:
    """Dense fp32 [rows, cols]: code * scale + min (the fused kernel's form)."""
    qblk, qsqm, ddm = qblk.contiguous(), qsqm.contiguous(), ddm.contiguous()
    out = torch.empty(rows, cols, dtype=torch.float32)
    rc = lib().rqo_sb6_dequantize(_p(qblk), _p(qsqm), _p(ddm.view(torch.int16)), rows, cols,
                                  gw_sb, xbits, _p(out))
    if rc != 0:
        raise ValueError(f"oracle sb6 dequantize rejected arguments (rc={rc})")
    return out

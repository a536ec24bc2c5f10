"""ctypes binding of librwkvq_hip.so (the C ABI in include/rwkvq.h).

torch is imported first on purpose: torch ships its own libamdhip64.so.7 and
loading it before the library makes the library bind to that same HIP
runtime (same soname), so torch's streams and device pointers are valid in
library calls.  There is no CPU path: if the library is missing the import
of the ops fails loudly.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must be loaded before the HIP library, see above)

# RWKVQ_LIB selects another build of the same ABI (e.g. a tuning variant).
LIB_PATH = os.environ.get("RWKVQ_LIB") or os.path.join(
    os.path.dirname(os.path.abspath(__file__)), "librwkvq_hip.so")

RQ_BF16, RQ_F16, RQ_F32 = 0, 1, 2
DTYPE_CODE = {torch.bfloat16: RQ_BF16, torch.float16: RQ_F16, torch.float32: RQ_F32}

# Every entry point the header declares, with its ctypes signature.
_i32, _i64, _vp = ctypes.c_int, ctypes.c_int64, ctypes.c_void_p


class RqProblem(ctypes.Structure):
    """Mirror of rq_problem."""

    _fields_ = [
        ("x", _vp),
        ("w_q", _vp),
        ("scales", _vp),
        ("biases", _vp),
        ("y", _vp),
        ("rows", _i64),
        ("cols", _i64),
    ]


class RqGroupedPlan(ctypes.Structure):
    """Mirror of rq_grouped_plan."""

    _fields_ = [("opaque", _i64 * 8)]


SIGNATURES = {
    "rq_abi_version": ([], _i32),
    "rq_last_error": ([], ctypes.c_char_p),
    "rq_quantize": ([_vp, _i32, _i64, _i64, _i32, _i32, _vp, _vp, _vp, _vp], _i32),
    "rq_dequantize": ([_vp, _vp, _vp, _i32, _i64, _i64, _i32, _i32, _vp, _i32, _vp], _i32),
    "rq_qmm": ([_vp, _i32, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i32, _i32, _i32, _vp, _i32, _vp],
               _i32),
    "rq_qmm_splitk_workspace_bytes": ([_i64, _i64, _i64, _i32, _i32], _i64),
    "rq_qmm_splitk": ([_vp, _i32, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i32, _i32, _vp, _i32,
                       _vp, _i64, _vp], _i32),
    "rq_qmm_lora": ([_vp, _i32, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i32, _i32, _i32, _vp, _vp,
                     _i64, ctypes.c_float, _vp, _i32, _vp], _i32),
    "rq_qlora": ([_vp, _i32, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i32, _i32, _i32, _vp, _vp,
                  _i64, ctypes.c_float, _vp, _vp, _i32, _vp], _i32),
    "rq_qlora_dx": ([_vp, _i32, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i32, _i32, _vp, _vp,
                     _i64, ctypes.c_float, _vp, _vp, _i32, _vp], _i32),
    "rq_lora_down": ([_vp, _i64, _i64, _vp, _i64, _vp, _vp], _i32),
    "rq_lora_grads_workspace_bytes": ([_i64, _i64, _i64, _i64, _i32, _i32], _i64),
    "rq_lora_grads": ([_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, ctypes.c_float, _vp, _vp, _vp,
                       _i64, _vp], _i32),
    "rq_lora_grads_f32": ([_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, ctypes.c_float, _vp, _vp,
                           _vp, _i64, _vp], _i32),
    "rq_lora_grads_noalloc": ([_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, ctypes.c_float, _vp,
                               _vp, _vp], _i32),
    "rq_embedding": ([_vp, _i64, _vp, _vp, _vp, _i32, _i64, _i64, _i32, _i32, _vp, _i32, _vp],
                     _i32),
    "rq_sb6_dequantize": ([_vp, _vp, _vp, _i64, _i64, _i32, _i32, _i32, _vp, _i32, _vp], _i32),
    "rq_sb6_to_affine": ([_vp, _vp, _vp, _i64, _i64, _i32, _i32, _i32, _vp, _vp, _vp, _vp], _i32),
    "rq_pack": ([_vp, _i64, _i64, _i32, _vp, _vp], _i32),
    "rq_unpack": ([_vp, _i64, _i64, _i32, _vp, _vp], _i32),
    "rq_qmm_grouped": ([ctypes.POINTER(RqProblem), _i32, _i32, _i32, _i32, _i64, _i32, _i32, _vp],
                       _i32),
    "rq_grouped_plan_table_bytes": ([ctypes.POINTER(RqProblem), _i32], _i64),
    "rq_grouped_plan_init": ([ctypes.POINTER(RqProblem), _i32, _i32, _i32, _i32, _i64, _i32, _i32,
                              _vp, _i64, ctypes.POINTER(RqGroupedPlan), _vp], _i32),
    "rq_grouped_plan_run": ([ctypes.POINTER(RqGroupedPlan), _vp], _i32),
}
RQ_EUNSUPPORTED = -4

ABI_VERSION = 1
MAX_GROUPED = 48

_lib = None


class RwkvqError(RuntimeError):
    """A non-zero return of the C ABI."""


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RwkvqError(
                f"librwkvq_hip.so not found at {LIB_PATH}; build it with "
                "`python rwkv-metal_amd/build_lib.py` (or __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        if L.rq_abi_version() != ABI_VERSION:
            raise RwkvqError(f"librwkvq_hip ABI {L.rq_abi_version()} != expected {ABI_VERSION}")
        _lib = L
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().rq_last_error().decode(errors="replace")
        if rc == -1:
            raise ValueError(f"{what}: {msg}")
        raise RwkvqError(f"{what} failed (rc={rc}): {msg}")

"""The C ABI library loads on a machine without a GPU, exports every entry
point include/rwkvq.h declares, and rejects bad arguments before touching the
device (no compute calls here)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "rwkvq.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(rq_\w+)\s*\(", text, flags=re.M)))


@pytest.fixture(scope="module")
def L():
    from rwkvq import _lib
    return _lib.lib()


def test_header_declares_the_expected_surface():
    assert declared_functions() == sorted([
        "rq_abi_version", "rq_last_error", "rq_quantize", "rq_dequantize", "rq_qmm",
        "rq_pack", "rq_unpack", "rq_qmm_grouped", "rq_grouped_plan_table_bytes",
        "rq_grouped_plan_init", "rq_grouped_plan_run", "rq_embedding", "rq_sb6_dequantize",
        "rq_sb6_to_affine", "rq_qmm_lora", "rq_lora_down", "rq_lora_grads_workspace_bytes",
        "rq_lora_grads", "rq_lora_grads_f32", "rq_lora_grads_noalloc", "rq_qlora",
        "rq_qlora_dx", "rq_qmm_splitk_workspace_bytes", "rq_qmm_splitk"])


def test_library_exports_every_declared_symbol(L):
    from rwkvq import _lib
    for name in declared_functions():
        assert hasattr(L, name), f"{name} missing from librwkvq_hip.so"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert L.rq_abi_version() == 1


def _err(L):
    return L.rq_last_error().decode()


def test_invalid_arguments_return_einval(L):
    p = 0x1000  # never dereferenced: validation fails first
    assert L.rq_qmm(p, 0, p, p, p, 0, 1, 64, 64, 64, 7, 1, p, 0, None) == -1
    assert "bits" in _err(L)
    assert L.rq_qmm(p, 0, p, p, p, 0, 1, 64, 64, 48, 4, 1, p, 0, None) == -1
    assert "group_size" in _err(L)
    assert L.rq_quantize(p, 0, 4, 96, 64, 4, p, p, p, None) == -1
    assert "divisible" in _err(L)
    assert L.rq_dequantize(p, p, p, 0, -1, 64, 64, 4, p, 0, None) == -1
    assert L.rq_qmm(p, 7, p, p, p, 0, 1, 64, 64, 64, 4, 1, p, 0, None) == -1
    assert L.rq_qmm(0, 0, p, p, p, 0, 1, 64, 64, 64, 4, 1, p, 0, None) == -1
    assert "NULL" in _err(L)
    assert L.rq_embedding(p, -1, p, p, p, 0, 8, 64, 64, 4, p, 0, None) == -1
    assert "negative" in _err(L)
    assert L.rq_embedding(0, 3, p, p, p, 0, 8, 64, 64, 4, p, 0, None) == -1
    assert "NULL" in _err(L)
    assert L.rq_embedding(p, 3, p, p, p, 0, 8, 64, 64, 7, p, 0, None) == -1
    assert L.rq_embedding(p, 0, p, p, p, 0, 8, 64, 64, 4, p, 0, None) == 0
    assert L.rq_sb6_dequantize(p, p, p, 4, 64, 64, 1, 2, p, 2, None) == -1
    assert "32 codes" in _err(L)
    assert L.rq_sb6_dequantize(p, p, p, 4, 64, 32, 1, 3, p, 2, None) == -1
    assert "xbits" in _err(L)
    assert L.rq_sb6_dequantize(p, p, p, 4, 96, 32, 2, 0, p, 2, None) == -1
    assert "gw_sb" in _err(L)
    assert L.rq_sb6_to_affine(p, p, p, 4, 64, 32, 1, 0, p, 0, p, None) == -1
    assert L.rq_sb6_to_affine(p + 1, p, p, 4, 64, 32, 1, 0, p, p, p, None) == -2
    assert L.rq_qmm_lora(p, 0, p, p, p, 0, 300, 64, 64, 64, 4, 1, p, p, 8, 1.0, p, 0, None) == -1
    assert "rank" in _err(L)
    assert L.rq_qmm_lora(p, 0, p, p, p, 0, 300, 64, 64, 64, 4, 1, 0, p, 16, 1.0, p, 0, None) == -1
    assert L.rq_qmm_lora(p, 0, p, p, p, 0, 300, 64, 64, 64, 4, 1, p + 8, p, 16, 1.0, p, 0, None) == -2
    assert L.rq_lora_down(p, 64, 64, p, 8, p, None) == -1
    assert "rank" in _err(L)
    assert L.rq_lora_down(p, 64, 48, p, 16, p, None) == -1
    assert "multiple of 32" in _err(L)
    assert L.rq_lora_down(p, 64, 64, 0, 16, p, None) == -1
    assert L.rq_lora_down(p + 8, 64, 64, p, 16, p, None) == -2
    assert L.rq_lora_down(p, 0, 64, p, 16, p, None) == 0  # nothing to do


def test_misaligned_pointers_return_ealign(L):
    p, odd = 0x1000, 0x1002
    assert L.rq_qmm(odd, 0, p, p, p, 0, 1, 64, 64, 64, 4, 1, p, 0, None) == -2
    assert L.rq_quantize(odd, 0, 4, 64, 64, 4, p, p, p, None) == -2
    assert L.rq_unpack(p, 4, 64, 4, odd, None) == -2


def test_empty_problems_are_no_ops(L):
    assert L.rq_quantize(0, 0, 0, 64, 64, 4, 0, 0, 0, None) == 0
    assert L.rq_dequantize(0, 0, 0, 0, 5, 0, 64, 4, 0, 0, None) == 0
    assert L.rq_qmm(0, 0, 0, 0, 0, 0, 0, 64, 64, 64, 4, 1, 0, 0, None) == 0
    assert L.rq_qmm_grouped(None, 0, 0, 0, 0, 1, 64, 4, None) == 0
    assert _err(L) == ""


def test_grouped_rejects_large_m(L):
    from rwkvq._lib import RqProblem
    probs = (RqProblem * 1)()
    assert L.rq_qmm_grouped(probs, 1, 0, 0, 0, 17, 64, 4, None) == -1
    assert "m must be" in _err(L)


def _problems(shapes, sb_align=0):
    from rwkvq._lib import RqProblem
    probs = (RqProblem * len(shapes))()
    for i, (R, K) in enumerate(shapes):
        probs[i] = RqProblem(0x1000, 0x2000, 0x3000 + sb_align, 0x4000, 0x5000, R, K)
    return probs


def test_plan_table_bytes(L):
    # descriptors (56 B each, padded to 16) + one uint32 per 64-row block
    probs = _problems([(2048, 2048), (65536, 2048), (100, 512)])
    assert L.rq_grouped_plan_table_bytes(probs, 3) == 176 + 4 * (32 + 1024 + 2)


def test_plan_rejections_before_any_device_work(L):
    from ctypes import byref
    from rwkvq._lib import RQ_EUNSUPPORTED, RqGroupedPlan
    plan = RqGroupedPlan()
    probs = _problems([(2048, 2048)])
    # fp32 scales are outside the planned kernel
    assert L.rq_grouped_plan_init(probs, 1, 0, 2, 2, 1, 64, 4, 0x10000, 1 << 20, byref(plan),
                                  None) == RQ_EUNSUPPORTED
    assert "rq_qmm_grouped" in _err(L)
    # cols not a multiple of 512
    probs = _problems([(2048, 768)])
    assert L.rq_grouped_plan_init(probs, 1, 0, 0, 0, 1, 64, 4, 0x10000, 1 << 20, byref(plan),
                                  None) == RQ_EUNSUPPORTED
    # misaligned scales
    probs = _problems([(2048, 2048)], sb_align=2)
    assert L.rq_grouped_plan_init(probs, 1, 0, 0, 0, 1, 64, 4, 0x10000, 1 << 20, byref(plan),
                                  None) == RQ_EUNSUPPORTED
    # table too small
    probs = _problems([(2048, 2048)])
    assert L.rq_grouped_plan_init(probs, 1, 0, 0, 0, 1, 64, 4, 0x10000, 16, byref(plan),
                                  None) == -1
    assert "needs" in _err(L)
    # a plan that was never initialised does not run
    assert L.rq_grouped_plan_run(byref(RqGroupedPlan()), None) == -1
    # an empty set is a valid plan whose run is a no-op
    assert L.rq_grouped_plan_init(None, 0, 0, 0, 0, 1, 64, 4, None, 0, byref(plan), None) == 0
    assert L.rq_grouped_plan_run(byref(plan), None) == 0


def test_lora_grads_workspace_and_rejections(L):
    """The gradient launch's workspace: none when one chunk per tile already
    fills the GPU, fp32 partial tiles plus one counter per tile otherwise;
    bad ranks, unaligned operands and a short workspace are refused."""
    p = 0x1000
    # 4096 rows, K = N = 2048, rank 16: 64 tiles, 8 chunks of 512 rows (~512 jobs)
    counters = 16384 * 4
    nb = L.rq_lora_grads_workspace_bytes(4096, 2048, 2048, 16, 1, 1)
    assert nb == counters + 64 * 8 * 64 * 16 * 4
    # only dB: 32 tiles, 16 chunks of 256 rows (64 rows per step, 64 steps)
    assert L.rq_lora_grads_workspace_bytes(4096, 2048, 2048, 16, 0, 1) == \
        counters + 32 * 16 * 64 * 16 * 4
    # few rows: one chunk, no workspace
    assert L.rq_lora_grads_workspace_bytes(64, 2048, 2048, 16, 1, 1) == 0
    # wide outputs at rank 64 stay within the 8 MiB partial cap
    nb = L.rq_lora_grads_workspace_bytes(4096, 8192, 8192, 64, 1, 1)
    assert 0 < nb <= (8 << 20) + counters
    assert L.rq_lora_grads_workspace_bytes(4096, 1 << 20, 8, 16, 1, 1) == -1
    assert L.rq_lora_grads_workspace_bytes(4096, 2048, 2048, 24, 1, 1) == -1
    assert L.rq_lora_grads(p, p, p, p, 4096, 2048, 2048, 24, 1.0, p, p, p, 1 << 30, None) == -1
    assert "rank" in _err(L)
    assert L.rq_lora_grads(p, p, p, p, 4096, 2044, 2048, 16, 1.0, p, p, p, 1 << 30, None) == -1
    assert L.rq_lora_grads(p + 8, p, p, p, 4096, 2048, 2048, 16, 1.0, p, p, p, 1 << 30, None) == -2
    assert L.rq_lora_grads(p, p, p, p, 4096, 2048, 2048, 16, 1.0, p, p, p, 64, None) == -1
    assert "workspace" in _err(L)
    # dA only: dY and z are not read, so they may be NULL
    assert L.rq_lora_grads(p, p, 0, 0, 4096, 2048, 2048, 16, 1.0, p, 0, 0, 0, None) == -1
    assert "workspace" in _err(L)
    # the fp32-operand form checks the same things and names itself
    assert L.rq_lora_grads_f32(p, p, p, p, 4096, 2048, 2048, 24, 1.0, p, p, p, 1 << 30, None) == -1
    assert "rq_lora_grads_f32" in _err(L) and "rank" in _err(L)
    assert L.rq_lora_grads_f32(p + 8, p, p, p, 4096, 2048, 2048, 16, 1.0, p, p, p, 1 << 30,
                               None) == -2
    assert L.rq_lora_grads_f32(p, p, p, p, 4096, 2048, 2048, 16, 1.0, p, p, p, 64, None) == -1
    assert "workspace" in _err(L)


def test_lora_grads_noalloc_rejections_before_any_device_work(L):
    p = 0x1000
    assert L.rq_lora_grads_noalloc(p, p, p, p, 4096, 1 << 20, 8, 16, 1.0, p, p, None) == -1
    assert "exceeds" in _err(L)
    assert L.rq_lora_grads_noalloc(p, p, p, p, 4096, 2048, 2048, 20, 1.0, p, p, None) == -1
    assert L.rq_lora_grads_noalloc(p, p + 4, p, p, 4096, 2048, 2048, 16, 1.0, p, p, None) == -2


def test_qmm_splitk_plan_and_rejections(L):
    """The split-K plan (host only): config 3's long contraction at M = 512 and
    2048 splits; the K = 2560 shapes, M = 4096 and small M do not (their
    workspace size is 0 and rq_qmm_splitk is then rq_qmm)."""
    nb = L.rq_qmm_splitk_workspace_bytes
    for m in (512, 2048):
        b = nb(m, 2560, 10240, 64, 4)
        assert b > 0 and b % (m * 2560 * 4) == 0, (m, b)
        assert 2 <= b // (m * 2560 * 4) <= 32
    for m, r, k in [(4096, 2560, 2560), (4096, 10240, 2560), (4096, 2560, 10240),
                    (2048, 2560, 2560), (512, 2560, 2560), (100, 2560, 10240)]:
        assert nb(m, r, k, 64, 4) == 0, (m, r, k)
    assert nb(512, 2560, 10240, 48, 4) == -1 and "group_size" in _err(L)
    assert nb(512, 2560, 10240, 64, 7) == -1
    assert nb(-1, 2560, 10240, 64, 4) == -1
    p = 0x1000
    # a split problem without enough workspace is refused before any launch
    assert L.rq_qmm_splitk(p, 0, p, p, p, 0, 512, 2560, 10240, 64, 4, p, 0, p, 64, None) == -1
    assert "workspace" in _err(L)
    need = nb(512, 2560, 10240, 64, 4)
    assert L.rq_qmm_splitk(p, 0, p, p, p, 0, 512, 2560, 10240, 64, 4, p, 0, p + 8, need,
                           None) == -2


def test_qlora_dx_rejections_before_any_device_work(L):
    """rq_qlora_dx validates before it launches: the rank, NULL adapters,
    alignment (16 bytes for dy, lora_b and u_out, which are read or written
    in 16-byte pieces; 2 for lora_a) and an empty contraction; an empty
    output is a no-op."""
    p = 0x1000
    f = L.rq_qlora_dx
    assert f(p, 0, p, p, p, 0, 512, 2048, 2048, 64, 4, p, p, 8, 1.0, p, p, 0, None) == -1
    assert "rank" in _err(L)
    assert f(p, 0, p, p, p, 0, 512, 2048, 2048, 64, 4, 0, p, 16, 1.0, p, p, 0, None) == -1
    assert "NULL" in _err(L)
    assert f(p + 8, 0, p, p, p, 0, 512, 2048, 2048, 64, 4, p, p, 16, 1.0, p, p, 0, None) == -2
    assert f(p, 0, p, p, p, 0, 512, 2048, 2048, 64, 4, p + 1, p, 16, 1.0, p, p, 0, None) == -2
    assert "2-byte" in _err(L)
    assert f(p, 0, p, p, p, 0, 512, 2048, 2048, 64, 4, p, p + 2, 16, 1.0, p, p, 0, None) == -2
    assert "lora_b" in _err(L)
    assert f(p, 0, p, p, p, 0, 512, 2048, 2048, 64, 4, p, p, 16, 1.0, p + 8, p, 0, None) == -2
    assert f(p, 0, p, p, p, 0, 512, 0, 2048, 64, 4, p, p, 16, 1.0, p, p, 0, None) == -1
    assert "contraction" in _err(L)
    assert f(p, 0, p, p, p, 0, 512, 2048, 2048, 64, 7, p, p, 16, 1.0, p, p, 0, None) == -1
    assert f(p, 0, p, p, p, 0, 0, 2048, 2048, 64, 4, p, p, 16, 1.0, p, p, 0, None) == 0

"""GPU parity: the HIP library (through the C ABI, via the torch ops) against
the CPU oracle on identical seeded inputs.

Bar: quantize codes/words, scales and biases bit-exact; pack/unpack
bit-exact; dequantize bit-exact to the oracle's MLX arithmetic (multiply and
add each rounded in the scales dtype); quantized_matmul within rel-err 1e-2
(bf16 operands, fp32 accumulation) -- Frobenius-relative and elementwise
against the largest reference magnitude -- of the oracle's product with the
weights s*q + b unrounded (weights="exact", the form of MLX's qmv).  The
oracle's other form, with dequantize()'s bf16-rounded weights, sits up to ~1%
from it on N(0, 0.02) weights (tests/test_oracle.py pins both).
"""
import pytest
import torch

pytestmark = pytest.mark.gpu

BITS = (2, 3, 4, 5, 6, 8)
GROUPS = (32, 64, 128)
TOL = 1e-2


def weights(R, K, seed, dtype=torch.bfloat16, std=0.02):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(R, K, generator=g) * std).to(dtype)


def acts(M, K, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed + 500)
    return torch.randn(M, K, generator=g).to(dtype)


def special_rows(K, dtype):
    rows = [
        torch.zeros(K),                                   # all-zero groups
        torch.full((K,), 0.37),                           # constant groups
        -torch.linspace(0.1, 2.0, K),                     # all negative
        torch.linspace(0.1, 2.0, K),                      # all positive
        torch.linspace(-1.0, 1.0, K),                     # exact ties at 2^b grids
        torch.randn(K, generator=torch.Generator().manual_seed(9)) * 1e3,
        torch.randn(K, generator=torch.Generator().manual_seed(10)) * 1e-5,
    ]
    r = torch.stack(rows)
    r[:, ::5] = 0.0
    r[0] = 0.0
    return r.to(dtype)


def rel_check(y, ref, tol=TOL, what=""):
    y, ref = y.detach().double().cpu(), ref.detach().double().cpu()
    assert y.shape == ref.shape, (what, y.shape, ref.shape)
    assert torch.isfinite(y).all(), what
    denom = ref.norm().item()
    if denom == 0:
        assert y.abs().max().item() == 0, what
        return
    fro = (y - ref).norm().item() / denom
    elem = (y - ref).abs().max().item() / ref.abs().max().item()
    assert fro <= tol and elem <= tol, f"{what}: frobenius rel-err {fro:.3e}, elementwise {elem:.3e}"


def bits_equal(a, b):
    a, b = a.detach().cpu().contiguous(), b.detach().cpu().contiguous()
    if a.dtype in (torch.bfloat16, torch.float16):
        return torch.equal(a.view(torch.int16), b.view(torch.int16))
    if a.dtype == torch.float32:
        return torch.equal(a.view(torch.int32), b.view(torch.int32))
    return torch.equal(a, b)


def say(*a):
    print(*a, flush=True)


# ------------------------------------------------------------ quantize

@pytest.mark.parametrize("bits", BITS)
def test_quantize_near_ties_bit_exact(O, rq, dev, bits):
    """The quantizer rounds an approximate quotient unless it lies within
    2^-11 of a half-integer, where it takes the IEEE division: groups whose
    values sit at k + 1/2 + delta steps of their own scale (delta from 0 to
    +-3e-4, a few steps out of range) must give the oracle's codes exactly."""
    g = torch.Generator().manual_seed(4242 + bits)
    nb = (1 << bits) - 1
    rows = []
    for _ in range(256):
        c = float(torch.exp(torch.empty(1).uniform_(-12, 4, generator=g)))
        off = float(torch.empty(1).uniform_(-2, 2, generator=g))
        k = torch.randint(-1, nb + 1, (64,), generator=g).double()
        delta = torch.tensor([0.0, 1e-7, -1e-7, 3e-6, -3e-6, 3e-5, -3e-5, 3e-4, -3e-4])[
            torch.randint(0, 9, (64,), generator=g)].double()
        v = (k + 0.5 + delta) * c + off
        v[0], v[1] = off, off + nb * c  # the group's extremes
        rows.append(v)
    w = torch.stack(rows).float()
    owq, os_, ob = O.quantize(w, 64, bits)
    wq, s, b = rq.quantize(w.to(dev), 64, bits)
    assert bits_equal(wq, owq), f"codes differ near ties at {bits} bits"
    assert bits_equal(s, os_) and bits_equal(b, ob)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("gs", GROUPS)
@pytest.mark.parametrize("bits", BITS)
def test_quantize_bit_exact(O, rq, dev, bits, gs, dtype):
    K = 512
    w = torch.cat([weights(57, K, 1000 * bits + gs, dtype), special_rows(K, dtype)])
    say(f"quantize bits={bits} gs={gs} dtype={dtype} shape={tuple(w.shape)}")
    wq, s, b = rq.quantize(w.to(dev), gs, bits)
    torch.cuda.synchronize()
    owq, os_, ob = O.quantize(w, gs, bits)
    assert torch.equal(wq.cpu(), owq), "packed words differ"
    assert bits_equal(s, os_) and bits_equal(b, ob), "scales/biases differ"
    assert torch.equal(rq.unpack_codes(wq, bits).cpu(), O.unpack(owq, bits))


def test_quantize_config1_shape(O, rq, dev):
    """benchmark config 1: RWKV-7 0.1B FFN key [3072, 768], 4-bit g64."""
    w = weights(3072, 768, 1_000_000 + 4)
    say("quantize config1 [3072,768]")
    wq, s, b = rq.quantize(w.to(dev), 64, 4)
    owq, os_, ob = O.quantize(w, 64, 4)
    assert torch.equal(wq.cpu(), owq) and bits_equal(s, os_) and bits_equal(b, ob)


# ------------------------------------------------------- pack / unpack

@pytest.mark.parametrize("bits", BITS)
def test_pack_unpack_bit_exact(O, rq, dev, bits):
    g = torch.Generator().manual_seed(bits)
    codes = torch.randint(0, 1 << bits, (37, 384), generator=g).to(torch.uint8)
    say(f"pack/unpack bits={bits}")
    wq = rq.pack_codes(codes.to(dev), bits)
    assert torch.equal(wq.cpu(), O.pack(codes, bits))
    assert torch.equal(rq.unpack_codes(wq, bits).cpu(), codes)


# ----------------------------------------------------------- dequantize

@pytest.mark.parametrize("sdt", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("gs", GROUPS)
@pytest.mark.parametrize("bits", BITS)
def test_dequantize_bit_exact(O, rq, dev, bits, gs, sdt):
    w = torch.cat([weights(45, 256, 77 * bits + gs, sdt), special_rows(256, sdt)])
    wq, s, b = O.quantize(w, gs, bits)
    say(f"dequantize bits={bits} gs={gs} sdt={sdt}")
    got = rq.dequantize(wq.to(dev), s.to(dev), b.to(dev), gs, bits)
    ref = O.dequantize(wq, s, b, gs, bits)
    assert got.dtype == sdt and bits_equal(got, ref)


# --------------------------------------------------------------- GEMV

@pytest.mark.parametrize("M", [1, 2, 5, 8, 16])
@pytest.mark.parametrize("gs", GROUPS)
@pytest.mark.parametrize("bits", BITS)
def test_qmv_parity_bf16(O, rq, dev, bits, gs, M):
    R, K = 200, 640
    w = weights(R, K, 31 * bits + gs)
    wq, s, b = O.quantize(w, gs, bits)
    x = acts(M, K, M + bits)
    say(f"qmv bits={bits} gs={gs} M={M}")
    y = rq.quantized_matmul(x.to(dev), wq.to(dev), s.to(dev), b.to(dev), True, gs, bits)
    ref = O.quantized_matmul(x, wq, s, b, True, gs, bits, out_dtype=torch.float32, weights="exact")
    assert y.dtype == torch.bfloat16
    rel_check(y, ref, what=f"qmv b{bits} g{gs} M{M}")


@pytest.mark.parametrize("xdt,sdt", [(torch.float32, torch.bfloat16), (torch.float32, torch.float32),
                                     (torch.float16, torch.float16), (torch.bfloat16, torch.float32)])
@pytest.mark.parametrize("bits,gs", [(4, 64), (4, 32), (6, 32), (3, 64), (8, 64), (5, 32)])
def test_qmv_parity_dtypes(O, rq, dev, bits, gs, xdt, sdt):
    """fp32 activations (the reference's default residual stream,
    rwkv_metal/model/rwkv7_x070.py:51) and fp32 scales at g32 (RwkvqNativeLinear,
    rwkv_metal/lora/rwkvq_native.py:119-122)."""
    R, K, M = 130, 512, 3
    w = weights(R, K, 5 * bits + gs, sdt)
    wq, s, b = O.quantize(w, gs, bits)
    x = acts(M, K, 8, xdt)
    say(f"qmv dtypes x={xdt} s={sdt} bits={bits} gs={gs}")
    y = rq.quantized_matmul(x.to(dev), wq.to(dev), s.to(dev), b.to(dev), True, gs, bits)
    want = xdt if xdt == sdt else torch.float32
    assert y.dtype == want
    ref = O.quantized_matmul(x, wq, s, b, True, gs, bits, out_dtype=torch.float32, weights="exact")
    rel_check(y, ref, what="qmv dtypes")


def _rel(y, ref):
    y, ref = y.detach().double().cpu(), ref.double()
    return ((y - ref).norm() / ref.norm()).item(), ((y - ref).abs().max() / ref.abs().max()).item()


# (R, K, gs, bits): small launches run the split GEMV (16-bit scales) or
# qmv_kernel (fp32 scales); 32768 rows run the streamed GEMV.
FP32_SHAPES = [(2048, 2048, 64, 4), (512, 4096, 32, 5), (4096, 2048, 64, 8), (32768, 1024, 64, 4),
               (32768, 512, 128, 3)]


@pytest.mark.parametrize("sdt", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("R,K,gs,bits", FP32_SHAPES)
def test_fp32_activation_precision(O, rq, dev, R, K, gs, bits, sdt):
    """fp32 activations (the reference's residual stream,
    rwkv_metal/model/rwkv7_x070.py:51; RwkvqNativeLinear casts x to fp32,
    rwkv_metal/lora/rwkvq_native.py:120).  At m <= 2 the decode GEMV multiplies
    x as its bf16 hi/lo split (bf16(x), bf16(x - bf16(x))) and adds the two
    products: within 1e-5 Frobenius / 3e-5 elementwise of MLX's fp32 product
    (the oracle's, in float64), where one bf16 rounding of x costs ~1.6e-3.
    Larger m (the wide GEMV at 8, the GEMM at 300) multiplies bf16(x) -- the
    GEMM also rounds each s*q + b to bf16 -- and stays within 3e-3 / 4e-3;
    the wide GEMV is the oracle's product of bf16(x) to fp32 summation
    order."""
    w = weights(R, K, R + K + bits, sdt)
    wq, s, b = O.quantize(w, gs, bits)
    g = torch.Generator().manual_seed(R + K + bits)
    for M in (1, 2, 8, 300):
        if M == 300 and R > 4096:
            continue  # the GEMM is covered at the smaller shapes
        say(f"fp32 activations [{R},{K}] b{bits} g{gs} s={sdt} M={M}")
        x = torch.randn(M, K, generator=g)
        y = rq.quantized_matmul(x.to(dev), wq.to(dev), s.to(dev), b.to(dev), True, gs, bits)
        assert y.dtype == torch.float32
        ref = O.quantized_matmul(x, wq, s, b, True, gs, bits, out_dtype=torch.float32, weights="exact")
        fro, elem = _rel(y, ref)
        if M <= 2:
            assert fro <= 1e-5 and elem <= 3e-5, f"M={M} vs fp32 x: {fro:.2e} {elem:.2e}"
            continue
        assert fro <= 3e-3 and elem <= 4e-3, f"M={M} vs fp32 x: {fro:.2e} {elem:.2e}"
        refb = O.quantized_matmul(x.to(torch.bfloat16).float(), wq, s, b, True, gs, bits,
                                  out_dtype=torch.float32, weights="exact")
        frob, elemb = _rel(y, refb)
        if M == 8:
            assert frob <= 1e-5 and elemb <= 2e-5, f"M={M} vs bf16(x): {frob:.2e} {elemb:.2e}"
        else:
            assert frob <= 2.5e-3, f"M={M} vs bf16(x): {frob:.2e}"


def test_fp16_and_planned_fp32_activations_exact(O, rq, dev):
    """The hi/lo split also carries f16 activations whole (11 significant
    bits; bf16 scales, so y is fp32), and the planned one-launch schedule
    (rq_grouped_plan_*) splits fp32 activations like single calls do."""
    wq, s, b = O.quantize(weights(4096, 2048, 77), 64, 4)
    for M in (1, 2):
        x = acts(M, 2048, 78 + M, torch.float16)
        say(f"f16 activations M={M}")
        y = rq.quantized_matmul(x.to(dev), wq.to(dev), s.to(dev), b.to(dev), True, 64, 4)
        assert y.dtype == torch.float32
        ref = O.quantized_matmul(x, wq, s, b, True, 64, 4, out_dtype=torch.float32, weights="exact")
        fro, elem = _rel(y, ref)
        assert fro <= 1e-5 and elem <= 3e-5, f"f16 M={M}: {fro:.2e} {elem:.2e}"
    probs = []
    for i in range(3):
        wq, s, b = O.quantize(weights(1024 * (i + 1), 1024, 90 + i), 64, 4)
        probs.append((wq, s, b))
    for M in (1, 2):
        xs = [torch.randn(M, 1024, generator=torch.Generator().manual_seed(95 + i)) for i in range(3)]
        plan = rq.GroupedQmv([x.to(dev) for x in xs], [(a.to(dev), c.to(dev), d.to(dev)) for a, c, d in probs],
                             64, 4, planned=True)
        assert plan.plan is not None
        ys = plan.run()
        torch.cuda.synchronize()
        for x, (wq, s, b), y in zip(xs, probs, ys):
            ref = O.quantized_matmul(x, wq, s, b, True, 64, 4, out_dtype=torch.float32, weights="exact")
            fro, elem = _rel(y, ref)
            assert fro <= 1e-5 and elem <= 3e-5, f"planned M={M}: {fro:.2e} {elem:.2e}"


# Small single launches (the K-split kernel) over contraction lengths from
# one 256-code stage to 16384, rows ending mid-tile.
SMALL_SHAPES = [(200, 256), (37, 768), (130, 2048), (64, 2304), (100, 8192), (17, 16384)]


@pytest.mark.parametrize("M", [1, 2, 4])
@pytest.mark.parametrize("gs", GROUPS)
@pytest.mark.parametrize("bits", BITS)
def test_qmv_small_launch_shapes(O, rq, dev, bits, gs, M):
    for R, K in SMALL_SHAPES:
        w = weights(R, K, 7 * bits + gs + K)
        wq, s, b = O.quantize(w, gs, bits)
        x = acts(M, K, M + K)
        say(f"qmv small bits={bits} gs={gs} M={M} R={R} K={K}")
        y = rq.quantized_matmul(x.to(dev), wq.to(dev), s.to(dev), b.to(dev), True, gs, bits)
        ref = O.quantized_matmul(x, wq, s, b, True, gs, bits, out_dtype=torch.float32, weights="exact")
        rel_check(y, ref, what=f"small b{bits} g{gs} M{M} {R}x{K}")


# The split GEMV (small launches: a block is one 16-row tile whose waves take
# contiguous K slices of 1, 2 or 4 256-code stages; m <= 4 in one pass of
# activation rows, 4 < m <= 8 in two).  Stage counts that do not divide into
# the slices leave the last wave a short slice: 9 stages on 9 waves of one,
# 17 / 21 on 2-stage slices, 33 / 63 on 4-stage slices.
SPLIT_SHAPES = [(37, 2304), (130, 4352), (16, 5376), (61, 8448), (200, 16128)]


@pytest.mark.parametrize("xdt,sdt", [(torch.bfloat16, torch.bfloat16), (torch.float16, torch.float16),
                                     (torch.float32, torch.bfloat16)])
@pytest.mark.parametrize("M", [1, 2, 3, 4, 6, 8])
@pytest.mark.parametrize("gs", GROUPS)
@pytest.mark.parametrize("bits", BITS)
def test_split_gemv_short_slices(O, rq, dev, bits, gs, M, xdt, sdt):
    for R, K in SPLIT_SHAPES:
        w = weights(R, K, 11 * bits + gs + K, sdt)
        wq, s, b = O.quantize(w, gs, bits)
        x = acts(M, K, 3 * M + K, xdt)
        say(f"split gemv bits={bits} gs={gs} M={M} x={xdt} R={R} K={K}")
        y = rq.quantized_matmul(x.to(dev), wq.to(dev), s.to(dev), b.to(dev), True, gs, bits)
        ref = O.quantized_matmul(x, wq, s, b, True, gs, bits, out_dtype=torch.float32, weights="exact")
        rel_check(y, ref, what=f"split b{bits} g{gs} M{M} {R}x{K}")


@pytest.mark.parametrize("M", [5, 8])
@pytest.mark.parametrize("bits", [4, 8])
def test_split_gemv_whole_cu_lds(O, rq, dev, bits, M):
    """Launches of at most one block per CU may stage up to 152 KB of x per
    block: [2048, 8192] at m = 8 runs 16 waves of 2-stage slices (4-bit
    codes; 8-bit codes at m > 4 take one stage per wave and fall back)."""
    for R, K in [(2048, 8192), (130, 4352), (256, 7936)]:
        w = weights(R, K, 70_000 + bits + K)
        wq, s, b = O.quantize(w, 64, bits)
        x = acts(M, K, 70_100 + M + K)
        say(f"split gemv whole-CU LDS bits={bits} M={M} R={R} K={K}")
        y = rq.quantized_matmul(x.to(dev), wq.to(dev), s.to(dev), b.to(dev), True, 64, bits)
        ref = O.quantized_matmul(x, wq, s, b, True, 64, bits, out_dtype=torch.float32, weights="exact")
        rel_check(y, ref, what=f"split whole-CU b{bits} M{M} {R}x{K}")


# Launches of at most 128 16-row tiles with K % 512 == 0 and bf16 x fold at
# m = 1, and at m = 2 when K >= 4096: W [R, K] runs as [2R, K/2] against x as
# [2m, K/2] and the store adds each output's two halves (m = 3, 4 and the
# shorter rows at m = 2 take the unfolded split GEMV on the same shapes).
FOLD_SHAPES = [(2048, 8192), (2048, 2048), (100, 4096), (37, 1024), (130, 512), (16, 16384)]


@pytest.mark.parametrize("M", [1, 2, 3, 4])
@pytest.mark.parametrize("gs", GROUPS)
@pytest.mark.parametrize("bits", BITS)
def test_split_gemv_fold(O, rq, dev, bits, gs, M):
    for R, K in FOLD_SHAPES:
        w = weights(R, K, 72_000 + 11 * bits + gs + K)
        wq, s, b = O.quantize(w, gs, bits)
        x = acts(M, K, 72_100 + 3 * M + K)
        say(f"split gemv fold bits={bits} gs={gs} M={M} R={R} K={K}")
        y = rq.quantized_matmul(x.to(dev), wq.to(dev), s.to(dev), b.to(dev), True, gs, bits)
        ref = O.quantized_matmul(x, wq, s, b, True, gs, bits, out_dtype=torch.float32, weights="exact")
        rel_check(y, ref, what=f"fold b{bits} g{gs} M{M} {R}x{K}")


def test_split_gemv_fold_grouped(O, rq, dev):
    """A folded grouped launch (two [512, 4096] problems and a [384, 4096]
    one, 88 tiles in all) against the oracle and bit-equal to single calls."""
    probs = []
    for i, R in enumerate((512, 512, 384)):
        wq, s, b = O.quantize(weights(R, 4096, 72_200 + i), 64, 4)
        probs.append((acts(2, 4096, 72_300 + i).to(dev), (wq.to(dev), s.to(dev), b.to(dev))))
    say("split gemv fold: grouped launch of 88 tiles")
    ys = rq.grouped_qmv([x for x, _ in probs], [w for _, w in probs], 64, 4)
    for (x, (wq, s, b)), y in zip(probs, ys):
        ref = O.quantized_matmul(x.cpu(), wq.cpu(), s.cpu(), b.cpu(), True, 64, 4,
                                 out_dtype=torch.float32, weights="exact")
        rel_check(y, ref, what="fold grouped")
        y1 = rq.grouped_qmv([x], [(wq, s, b)], 64, 4)[0]
        assert bits_equal(y, y1)


def test_split_gemv_whole_cu_boundary(O, rq, dev):
    """84 KB of staged x per block at m = 8 (K = 4352: 9 waves of 2-stage
    slices): 4096 rows (256 blocks) take the split GEMV with its larger LDS
    budget, 4112 rows (257 blocks) another kernel; a grouped launch of three
    problems with 255 blocks in all takes the split GEMV.  Every output row
    against the oracle, and the grouped launch bit-equal to single calls."""
    K = 4352
    for R in (4096, 4112):
        wq, s, b = O.quantize(weights(R, K, 71_000 + R), 64, 4)
        x = acts(8, K, 71_100 + R)
        say(f"split gemv whole-CU boundary R={R} K={K} M=8")
        y = rq.quantized_matmul(x.to(dev), wq.to(dev), s.to(dev), b.to(dev), True, 64, 4)
        ref = O.quantized_matmul(x, wq, s, b, True, 64, 4, out_dtype=torch.float32, weights="exact")
        rel_check(y, ref, what=f"whole-CU boundary {R}x{K}")
    probs = []
    for i, R in enumerate((1360, 1360, 1352)):
        wq, s, b = O.quantize(weights(R, K, 71_200 + i), 64, 4)
        probs.append((acts(8, K, 71_300 + i).to(dev), (wq.to(dev), s.to(dev), b.to(dev))))
    say("split gemv whole-CU boundary: grouped launch of 255 blocks")
    ys = rq.grouped_qmv([x for x, _ in probs], [w for _, w in probs], 64, 4)
    for (x, (wq, s, b)), y in zip(probs, ys):
        ref = O.quantized_matmul(x.cpu(), wq.cpu(), s.cpu(), b.cpu(), True, 64, 4,
                                 out_dtype=torch.float32, weights="exact")
        rel_check(y, ref, what="whole-CU boundary grouped")
        assert bits_equal(y, rq.quantized_matmul(x, wq, s, b, True, 64, 4))


def test_split_gemv_dependency_level(O, rq, dev):
    """One decode dependency level as one grouped launch (the r, k, v
    projections of a layer: three problems, three activations) and the
    same problems again as single calls: bit-identical, since each row's
    slices are summed in the same order."""
    probs = []
    for i in range(3):
        wq, s, b = O.quantize(weights(2048, 2048, 60_000 + i), 64, 4)
        probs.append((acts(1, 2048, 60_100 + i).to(dev), (wq.to(dev), s.to(dev), b.to(dev))))
    ys = rq.grouped_qmv([x for x, _ in probs], [w for _, w in probs], 64, 4)
    for (x, (wq, s, b)), y in zip(probs, ys):
        ref = O.quantized_matmul(x.cpu(), wq.cpu(), s.cpu(), b.cpu(), True, 64, 4,
                                 out_dtype=torch.float32, weights="exact")
        rel_check(y, ref, what="dependency level")
        y1 = rq.quantized_matmul(x, wq, s, b, True, 64, 4)
        assert bits_equal(y, y1)


def test_qmv_edge_shapes(O, rq, dev):
    cases = [(1, 32, 32, 4, 1), (17, 96, 32, 3, 4), (5, 160, 32, 6, 7), (33, 128, 128, 8, 16),
             (1, 64, 64, 2, 1), (250, 96, 32, 5, 3)]
    for R, K, gs, bits, M in cases:
        w = weights(R, K, R + K)
        wq, s, b = O.quantize(w, gs, bits)
        x = acts(M, K, R)
        say(f"qmv edge R={R} K={K} gs={gs} bits={bits} M={M}")
        y = rq.quantized_matmul(x.to(dev), wq.to(dev), s.to(dev), b.to(dev), True, gs, bits)
        ref = O.quantized_matmul(x, wq, s, b, True, gs, bits, out_dtype=torch.float32, weights="exact")
        rel_check(y, ref, what=f"edge {R}x{K}")


# --------------------------------------------------------------- GEMM

@pytest.mark.parametrize("M", [17, 100, 300])
@pytest.mark.parametrize("gs", GROUPS)
@pytest.mark.parametrize("bits", BITS)
def test_qmm_t_parity(O, rq, dev, bits, gs, M):
    R, K = 200, 384
    w = weights(R, K, 13 * bits + gs)
    wq, s, b = O.quantize(w, gs, bits)
    x = acts(M, K, M)
    say(f"qmm_t bits={bits} gs={gs} M={M}")
    y = rq.quantized_matmul(x.to(dev), wq.to(dev), s.to(dev), b.to(dev), True, gs, bits)
    ref = O.quantized_matmul(x, wq, s, b, True, gs, bits, out_dtype=torch.float32, weights="exact")
    rel_check(y, ref, what=f"qmm_t b{bits} g{gs} M{M}")


@pytest.mark.parametrize("M", [1, 8, 33, 200])
@pytest.mark.parametrize("gs", GROUPS)
@pytest.mark.parametrize("bits", BITS)
def test_qmm_n_parity(O, rq, dev, bits, gs, M):
    """transpose=False: dX = dY . W, the QLoRA backward through a frozen base."""
    R, K = 136, 384
    w = weights(R, K, 17 * bits + gs)
    wq, s, b = O.quantize(w, gs, bits)
    dy = acts(M, R, M + 1)
    say(f"qmm_n bits={bits} gs={gs} M={M}")
    y = rq.quantized_matmul(dy.to(dev), wq.to(dev), s.to(dev), b.to(dev), False, gs, bits)
    ref = O.quantized_matmul(dy, wq, s, b, False, gs, bits, out_dtype=torch.float32, weights="exact")
    rel_check(y, ref, what=f"qmm_n b{bits} g{gs} M{M}")


@pytest.mark.parametrize("M", [256, 300])
@pytest.mark.parametrize("gs", GROUPS)
@pytest.mark.parametrize("bits", BITS)
def test_qmm_n_warp_specialised_parity(O, rq, dev, bits, gs, M):
    """transpose=False at M >= 256 with R % 64 == 0 and K % 128 == 0: the
    warp-specialised kernel (partial M tile at M=300)."""
    R, K = 192, 384
    w = weights(R, K, 19 * bits + gs)
    wq, s, b = O.quantize(w, gs, bits)
    dy = acts(M, R, M + 3)
    say(f"qmm_n ws bits={bits} gs={gs} M={M}")
    y = rq.quantized_matmul(dy.to(dev), wq.to(dev), s.to(dev), b.to(dev), False, gs, bits)
    ref = O.quantized_matmul(dy, wq, s, b, False, gs, bits, out_dtype=torch.float32, weights="exact")
    rel_check(y, ref, what=f"qmm_n ws b{bits} g{gs} M{M}")


@pytest.mark.parametrize("M", [256, 300])
@pytest.mark.parametrize("gs", GROUPS)
@pytest.mark.parametrize("bits", BITS)
def test_qmm_t_k64_parity(O, rq, dev, bits, gs, M):
    """transpose=True at M >= 256 with whole 8-group chunks: the 64-wide-stage
    warp-specialised kernel (partial M and N tiles)."""
    R, K = 200, 8 * gs * 2
    w = weights(R, K, 23 * bits + gs)
    wq, s, b = O.quantize(w, gs, bits)
    x = acts(M, K, M + 5)
    say(f"qmm_t k64 bits={bits} gs={gs} M={M}")
    y = rq.quantized_matmul(x.to(dev), wq.to(dev), s.to(dev), b.to(dev), True, gs, bits)
    ref = O.quantized_matmul(x, wq, s, b, True, gs, bits, out_dtype=torch.float32, weights="exact")
    rel_check(y, ref, what=f"qmm_t k64 b{bits} g{gs} M{M}")


@pytest.mark.parametrize("transpose,R", [(True, 200), (True, 203), (True, 320), (False, 192)])
@pytest.mark.parametrize("sdt", [torch.bfloat16, torch.float16])
def test_qmm_k64_output_tiles(O, rq, dev, transpose, R, sdt):
    """The 64-wide-stage GEMMs' staged output stores: bf16 outputs (bf16
    scales) and fp32 outputs (bf16 x with f16 scales promote to fp32), whole
    and partial tiles in both dims, and an output row length that is not a
    multiple of 8 (R=203: element-wise tail stores)."""
    gs, bits, M = 64, 4, 300
    K = 8 * gs * 2
    w = weights(R, K, 29 + R, dtype=sdt)
    wq, s, b = O.quantize(w, gs, bits)
    x = acts(M, K if transpose else R, R + 7)
    say(f"qmm k64 tiles transpose={transpose} R={R} sdt={sdt}")
    y = rq.quantized_matmul(x.to(dev), wq.to(dev), s.to(dev), b.to(dev), transpose, gs, bits)
    assert y.dtype == (torch.bfloat16 if sdt == torch.bfloat16 else torch.float32)
    ref = O.quantized_matmul(x, wq, s, b, transpose, gs, bits, out_dtype=torch.float32,
                             weights="exact")
    rel_check(y, ref, what=f"qmm k64 tiles t{transpose} R{R} {sdt}")
    # every output element is written: compare against the oracle element-wise
    err = (y.double().cpu() - ref.double()).abs()
    assert (err <= 1e-2 * ref.double().abs().max() + 1e-3).all()


def test_qmm_t_k64_tile_order_covers_every_tile(rq, dev):
    """256 x 160 tiles walked in pairs of row tiles per column: M = 1200 gives
    5 row tiles (the last pair holds one) by 64 column tiles.  Every output
    element against an fp32 product of the HIP-dequantized weights."""
    M, R, K, gs, bits = 1200, 10240, 2560, 64, 4
    w = weights(R, K, 31).to(dev)
    wq, s, b = rq.quantize(w, gs, bits)
    x = acts(M, K, 37).to(dev)
    say(f"qmm_t k64 tile order M={M} R={R} K={K}")
    y = rq.quantized_matmul(x, wq, s, b, True, gs, bits)
    ref = x.float() @ rq.dequantize(wq, s, b, gs, bits).float().t()
    rel_check(y, ref, what="qmm_t k64 tile order")
    err = (y.float() - ref).abs()
    assert bool((err <= 1e-2 * ref.abs().max() + 1e-3).all())


@pytest.mark.parametrize("gs", GROUPS)
@pytest.mark.parametrize("bits", BITS)
def test_qmm_t_k64_256_row_tiles(O, rq, dev, bits, gs):
    """The 256-row tiles of the 64-wide-stage GEMM (eight MFMA waves of 64 x
    BN/2 beside four producer waves) for every bit width and group size: M =
    1100 gives 5 row tiles, the last one partial, by 64 (160-column, 4-bit) or
    80 column tiles.  Every output element against an fp32 product of the
    weights s*q + b from the bit-exact unpacked codes."""
    M, R, K = 1100, 10240, 16 * gs
    w = weights(R, K, 41 * bits + gs).to(dev)
    wq, s, b = rq.quantize(w, gs, bits)
    x = acts(M, K, 43 * bits + gs).to(dev)
    say(f"qmm_t k64 256-row tiles bits={bits} gs={gs}")
    y = rq.quantized_matmul(x, wq, s, b, True, gs, bits)
    ref = _gpu_dense_ref(rq, x, wq, s, b, gs, bits, True)
    rel_check(y, ref, what=f"qmm_t k64 256-row b{bits} g{gs}")
    err = (y.float() - ref).abs()
    assert bool((err <= 1e-2 * ref.abs().max() + 1e-3).all())


def test_qmm_t_k64_256_row_tiles_oracle(O, rq, dev):
    """One 256-row-tile problem against the CPU oracle itself (M = 800: 4 row
    tiles by 64 column tiles of 160)."""
    M, R, K = 800, 10240, 512
    w = weights(R, K, 47)
    wq, s, b = O.quantize(w, 64, 4)
    x = acts(M, K, 53)
    say("qmm_t k64 256-row tiles vs oracle")
    y = rq.quantized_matmul(x.to(dev), wq.to(dev), s.to(dev), b.to(dev), True, 64, 4)
    rel_check(y, O.quantized_matmul(x, wq, s, b, True, 64, 4, out_dtype=torch.float32,
                                    weights="exact"), what="k64 256-row oracle")


# split-K prefill (rq_qmm_splitk, routed by quantized_matmul where its plan
# splits): config 3's long contraction at M = 512 / 2048, a partial row tile
# with fp32 x, 3- and 8-bit codes, group sizes 32 / 128, f16 scales
SPLITK_CASES = [
    (512, 2560, 10240, 4, 64, torch.bfloat16, torch.bfloat16),
    (2048, 2560, 10240, 4, 64, torch.bfloat16, torch.bfloat16),
    (600, 2560, 10240, 4, 64, torch.bfloat16, torch.float32),
    (512, 2048, 16384, 3, 64, torch.bfloat16, torch.bfloat16),
    (512, 2048, 8192, 8, 32, torch.float16, torch.bfloat16),
    (512, 2560, 10240, 4, 128, torch.bfloat16, torch.bfloat16),
]


@pytest.mark.parametrize("M,R,K,bits,gs,sdt,xdt", SPLITK_CASES)
def test_qmm_splitk(rq, dev, M, R, K, bits, gs, sdt, xdt):
    """Every output element against an fp32 dense product; the split path is
    the one that runs, is deterministic (two calls, the same bits) and agrees
    with the unsplit rq_qmm within the bar."""
    from rwkvq._lib import DTYPE_CODE, lib
    from rwkvq.ops import _stream_on
    L = lib()
    nb = L.rq_qmm_splitk_workspace_bytes(M, R, K, gs, bits)
    assert nb > 0, "the plan must split this problem"
    say(f"splitk M={M} R={R} K={K} b={bits} gs={gs} s={sdt} x={xdt} ({nb // (M * R * 4)} splits)")
    wq, s, b = rq.quantize(weights(R, K, 96_000 + R + K + bits, sdt).to(dev), gs, bits)
    x = acts(M, K, 97_000 + M + bits, xdt).to(dev)
    y = rq.quantized_matmul(x, wq, s, b, True, gs, bits)
    y2 = rq.quantized_matmul(x, wq, s, b, True, gs, bits)
    assert bits_equal(y, y2), "split-K is not deterministic"
    ref = _gpu_dense_ref(rq, x, wq, s, b, gs, bits, True)
    rel_check(y, ref, what=f"splitk M{M} [{R},{K}] b{bits}")
    err = (y.float() - ref).abs()
    assert bool((err <= 1e-2 * ref.abs().max() + 1e-3).all())
    # the unsplit kernel on the same inputs
    yp = torch.empty_like(y)
    rc = L.rq_qmm(x.data_ptr(), DTYPE_CODE[x.dtype], wq.data_ptr(), s.data_ptr(), b.data_ptr(),
                  DTYPE_CODE[s.dtype], M, R, K, gs, bits, 1, yp.data_ptr(), DTYPE_CODE[yp.dtype],
                  _stream_on(dev))
    assert rc == 0, L.rq_last_error().decode()
    rel_check(y, yp.float(), what="splitk vs unsplit")
    # BoundQmm takes the same path with its own workspace
    bound = rq.BoundQmm(x, wq, s, b, True, gs, bits)
    assert bits_equal(bound.run(), y)


def test_qmm_splitk_oracle(O, rq, dev):
    """A split problem against the CPU oracle itself (M = 300: a partial row
    tile; K = 8192 in 16 shares)."""
    from rwkvq._lib import lib
    M, R, K = 300, 1280, 8192
    assert lib().rq_qmm_splitk_workspace_bytes(M, R, K, 64, 4) > 0
    w = weights(R, K, 98)
    wq, s, b = O.quantize(w, 64, 4)
    x = acts(M, K, 99)
    say("splitk vs oracle")
    y = rq.quantized_matmul(x.to(dev), wq.to(dev), s.to(dev), b.to(dev), True, 64, 4)
    rel_check(y, O.quantized_matmul(x, wq, s, b, True, 64, 4, out_dtype=torch.float32,
                                    weights="exact"), what="splitk oracle")


@pytest.mark.parametrize("R", [130, 77, 64])
def test_qmm_n_unaligned_rows(O, rq, dev, R):
    """Row counts whose activation rows are not 16-byte multiples (scalar loads)."""
    K, gs, bits = 256, 64, 4
    w = weights(R, K, R)
    wq, s, b = O.quantize(w, gs, bits)
    for xdt in (torch.bfloat16, torch.float32):
        dy = acts(45, R, R, xdt)
        say(f"qmm_n unaligned R={R} x={xdt}")
        y = rq.quantized_matmul(dy.to(dev), wq.to(dev), s.to(dev), b.to(dev), False, gs, bits)
        ref = O.quantized_matmul(dy, wq, s, b, False, gs, bits, out_dtype=torch.float32, weights="exact")
        rel_check(y, ref, what=f"qmm_n R{R}")


@pytest.mark.parametrize("xdt", [torch.float32, torch.float16])
def test_qmm_t_other_dtypes(O, rq, dev, xdt):
    R, K, M, gs, bits = 192, 256, 70, 32, 5
    w = weights(R, K, 3, torch.float32 if xdt == torch.float32 else xdt)
    wq, s, b = O.quantize(w, gs, bits)
    x = acts(M, K, 2, xdt)
    say(f"qmm_t x={xdt}")
    y = rq.quantized_matmul(x.to(dev), wq.to(dev), s.to(dev), b.to(dev), True, gs, bits)
    ref = O.quantized_matmul(x, wq, s, b, True, gs, bits, out_dtype=torch.float32, weights="exact")
    rel_check(y, ref, what="qmm_t dtypes")


# ---------------------------------------------------- benchmark configs

@pytest.mark.parametrize("M", [1, 16])
def test_config1_roundtrip_and_matmul(O, rq, dev, M):
    """0.1B FFN key [3072, 768] 4-bit g64: quantize -> unpack -> dequant -> y = x.Wq^T."""
    w = weights(3072, 768, 1_000_000 + 4)
    x = acts(M, 768, 1_000_000 + 4)
    say(f"config1 M={M}")
    wq, s, b = rq.quantize(w.to(dev), 64, 4)
    owq, os_, ob = O.quantize(w, 64, 4)
    assert torch.equal(wq.cpu(), owq)
    assert torch.equal(rq.unpack_codes(wq, 4).cpu(), O.unpack(owq, 4))
    assert bits_equal(rq.dequantize(wq, s, b, 64, 4), O.dequantize(owq, os_, ob, 64, 4))
    y = rq.quantized_matmul(x.to(dev), wq, s, b, True, 64, 4)
    rel_check(y, O.quantized_matmul(x, owq, os_, ob, True, 64, 4, out_dtype=torch.float32, weights="exact"))


CONFIG2 = {"r": (2048, 2048), "ffn_key": (8192, 2048), "ffn_value": (2048, 8192),
           "head": (65536, 2048)}


@pytest.mark.parametrize("M", [1, 8])
@pytest.mark.parametrize("name", list(CONFIG2))
def test_config2_decode_shapes(O, rq, dev, name, M):
    R, K = CONFIG2[name]
    w = weights(R, K, 2_000_000 + 6)
    wq, s, b = O.quantize(w, 64, 4)
    x = acts(M, K, 2_000_000 + 6)
    say(f"config2 {name} M={M}")
    y = rq.quantized_matmul(x.to(dev), wq.to(dev), s.to(dev), b.to(dev), True, 64, 4)
    ref = O.quantized_matmul(x, wq, s, b, True, 64, 4, out_dtype=torch.float32, weights="exact")
    rel_check(y, ref, what=f"config2 {name}")


def _gpu_dense_ref(rq, x, wq, s, b, gs, bits, transpose):
    """fp32 dense product with the weights s*q + b from the (bit-exact)
    unpacked codes -- the oracle's weights="exact" form, at sizes the CPU
    oracle is too slow for."""
    q = rq.unpack_codes(wq, bits).float()
    wd = q * s.float().repeat_interleave(gs, 1) + b.float().repeat_interleave(gs, 1)
    return x.float() @ (wd.t() if transpose else wd)


@pytest.mark.parametrize("M", [512, 2000, 2048, 4000, 4096])
@pytest.mark.parametrize("shape", [(2560, 2560), (10240, 2560), (2560, 10240)])
def test_config3_prefill_full_size(rq, dev, shape, M):
    """2.9B prefill shapes at full size.  The oracle is too slow here, so the
    reference is an fp32 matmul of the dequantized weights (dequantize is
    bit-exact to the oracle) -- a size-independent consistency check.  The
    2560-wide shapes run 64 x 96 tiles at M = 512 (the last column tile
    partial: 2560 = 26 * 96 + 64), 128-row tiles at M = 2000 / 2048, and
    256-row ones above; M = 2000 / 4000 end in a partial row tile."""
    R, K = shape
    say(f"config3 {shape} M={M}")
    w = weights(R, K, 3_000_000 + R).to(dev)
    wq, s, b = rq.quantize(w, 64, 4)
    x = acts(M, K, 3_000_000 + M).to(dev)
    y = rq.quantized_matmul(x, wq, s, b, True, 64, 4)
    rel_check(y, _gpu_dense_ref(rq, x, wq, s, b, 64, 4, True), what=f"config3 {shape} M{M}")


def test_config3_oracle_small_m(O, rq, dev):
    R, K, M = 2560, 2560, 512
    w = weights(R, K, 3_000_000 + R)
    wq, s, b = O.quantize(w, 64, 4)
    x = acts(M, K, 3_000_512)
    say("config3 oracle M=512")
    y = rq.quantized_matmul(x.to(dev), wq.to(dev), s.to(dev), b.to(dev), True, 64, 4)
    rel_check(y, O.quantized_matmul(x, wq, s, b, True, 64, 4, out_dtype=torch.float32, weights="exact"))


# The transposed GEMM's 160-column tiles: output widths that 128 does not
# divide (480, 800, 960) against the oracle, with partial row tiles and
# 40-code producer chunks spanning two or three groups (gs 32 / 64), and the
# 2.9B shapes at full size: 2560-wide outputs take 160 (256 tiles, one round,
# instead of 320), the 10240-wide one stays on 128.
N160_ORACLE = [(300, 128, 480, 4, 32, torch.bfloat16), (257, 192, 960, 8, 64, torch.float16),
               (512, 64, 800, 4, 32, torch.bfloat16), (700, 320, 960, 4, 64, torch.bfloat16)]


@pytest.mark.parametrize("M,R,K,bits,gs,sdt", N160_ORACLE)
def test_qmm_n_160_tiles_oracle(O, rq, dev, M, R, K, bits, gs, sdt):
    say(f"qmm_n 160 tiles M={M} R={R} K={K} bits={bits} gs={gs}")
    wq, s, b = O.quantize(weights(R, K, 80_000 + K + bits, sdt), gs, bits)
    dy = acts(M, R, 80_000 + M)
    y = rq.quantized_matmul(dy.to(dev), wq.to(dev), s.to(dev), b.to(dev), False, gs, bits)
    ref = O.quantized_matmul(dy, wq, s, b, False, gs, bits, out_dtype=torch.float32, weights="exact")
    rel_check(y, ref, what=f"qmm_n 160 {M}x{R}x{K}")


@pytest.mark.parametrize("M,R,K,bits,gs", [(4096, 2560, 2560, 4, 64), (4096, 10240, 2560, 4, 128),
                                           (4000, 2560, 2560, 8, 64), (2048, 2560, 10240, 4, 64)])
def test_config3_transposed_full_size(rq, dev, M, R, K, bits, gs):
    say(f"config3 transposed M={M} [{R},{K}] bits={bits} gs={gs}")
    wq, s, b = rq.quantize(weights(R, K, 3_100_000 + R + K).to(dev), gs, bits)
    dy = acts(M, R, 3_100_000 + M).to(dev)
    y = rq.quantized_matmul(dy, wq, s, b, False, gs, bits)
    rel_check(y, _gpu_dense_ref(rq, dy, wq, s, b, gs, bits, False), what=f"config3 dX {R}x{K} M{M}")


@pytest.mark.parametrize("shape", [(2048, 2048), (8192, 2048), (2048, 8192)])
def test_config4_transposed_full_size(rq, dev, shape):
    """QLoRA backward dX = dY . W at D=2048, M = 8 x 512."""
    R, K = shape
    say(f"config4 dX {shape}")
    w = weights(R, K, 4_000_000 + R).to(dev)
    wq, s, b = rq.quantize(w, 64, 4)
    dy = acts(4096, R, 4_000_800).to(dev)
    dx = rq.quantized_matmul(dy, wq, s, b, False, 64, 4)
    rel_check(dx, _gpu_dense_ref(rq, dy, wq, s, b, 64, 4, False), what=f"config4 {shape}")


@pytest.mark.parametrize("name,R,K,bits", [("proj", 4096, 4096, 3), ("ffn_key", 16384, 4096, 3),
                                           ("ffn_value", 4096, 16384, 3),
                                           ("head", 65536, 4096, 8)])
def test_config5_mixed_bits(O, rq, dev, name, R, K, bits):
    """7.2B shapes: 3-bit body (codes straddle words), 8-bit head; M=1 vs the
    oracle, M=2048 vs the dequantized fp32 reference."""
    say(f"config5 {name}")
    w = weights(R, K, 5_000_000 + R + bits)
    wq, s, b = O.quantize(w, 64, bits)
    gq, gs_, gb = rq.quantize(w.to(dev), 64, bits)
    assert torch.equal(gq.cpu(), wq) and bits_equal(gs_, s) and bits_equal(gb, b)
    x1 = acts(1, K, 5_000_500)
    y1 = rq.quantized_matmul(x1.to(dev), gq, gs_, gb, True, 64, bits)
    rel_check(y1, O.quantized_matmul(x1, wq, s, b, True, 64, bits, out_dtype=torch.float32, weights="exact"))
    x = acts(2048, K, 5_000_501).to(dev)
    y = rq.quantized_matmul(x, gq, gs_, gb, True, 64, bits)
    rel_check(y, _gpu_dense_ref(rq, x, gq, gs_, gb, 64, bits, True), what=f"config5 {name}")


# ------------------------------------------------------ grouped launch

def test_grouped_matches_single_calls(O, rq, dev):
    shapes = [(2048, 2048)] * 4 + [(8192, 2048), (2048, 8192), (300, 640)]
    xs, ws, refs = [], [], []
    for i, (R, K) in enumerate(shapes):
        w = weights(R, K, 60 + i)
        wq, s, b = O.quantize(w, 64, 4)
        x = acts(8, K, 60 + i)
        xs.append(x.to(dev))
        ws.append((wq.to(dev), s.to(dev), b.to(dev)))
        refs.append(O.quantized_matmul(x, wq, s, b, True, 64, 4, out_dtype=torch.float32, weights="exact"))
    say("grouped qmv")
    ys = rq.grouped_qmv(xs, ws, 64, 4)
    for y, ref, x, (wq, s, b) in zip(ys, refs, xs, ws):
        rel_check(y, ref, what="grouped")
        single = rq.quantized_matmul(x, wq, s, b, True, 64, 4)
        assert torch.allclose(y.float(), single.float(), rtol=1e-2, atol=1e-3)


def test_grouped_more_problems_than_one_launch(O, rq, dev):
    n = 70   # > RQ_MAX_GROUPED descriptors: two launches
    xs, ws, refs = [], [], []
    for i in range(n):
        w = weights(64, 256, 900 + i)
        wq, s, b = O.quantize(w, 64, 4)
        x = acts(1, 256, 900 + i)
        xs.append(x.to(dev))
        ws.append((wq.to(dev), s.to(dev), b.to(dev)))
        refs.append(O.quantized_matmul(x, wq, s, b, True, 64, 4, out_dtype=torch.float32, weights="exact"))
    say("grouped qmv, 70 problems")
    for y, ref in zip(rq.grouped_qmv(xs, ws, 64, 4), refs):
        rel_check(y, ref, what="grouped70")


# ------------------------------------------- planned (one-launch) grouped GEMV

# the streamed kernel's (scale, bias) windows cover 32 groups: 1536 and 2560
# columns end in a partial window (and, at 64-code groups, mid-iteration pair)
PLAN_SHAPES = [(100, 512), (64, 1024), (17, 2048), (24, 1536), (40, 2560)]


def _planned(O, rq, dev, shapes, M, gs, bits, seed, xdt=torch.bfloat16, sdt=torch.bfloat16):
    xs, ws, refs = [], [], []
    for i, (R, K) in enumerate(shapes):
        w = weights(R, K, seed + i, sdt)
        wq, s, b = O.quantize(w, gs, bits)
        x = acts(M, K, seed + i, xdt)
        xs.append(x.to(dev))
        ws.append((wq.to(dev), s.to(dev), b.to(dev)))
        refs.append(O.quantized_matmul(x, wq, s, b, True, gs, bits, out_dtype=torch.float32, weights="exact"))
    plan = rq.GroupedQmv(xs, ws, gs, bits, planned=True)
    assert plan.plan is not None
    return plan, refs, xs, ws


@pytest.mark.parametrize("M", [1, 2, 3, 4])
@pytest.mark.parametrize("gs", GROUPS)
@pytest.mark.parametrize("bits", BITS)
def test_planned_qmv_parity(O, rq, dev, bits, gs, M):
    say(f"planned qmv bits={bits} gs={gs} M={M}")
    plan, refs, _, _ = _planned(O, rq, dev, PLAN_SHAPES, M, gs, bits, 5000 + 10 * bits + gs)
    for y, ref in zip(plan.run(), refs):
        rel_check(y, ref, what=f"planned b{bits} g{gs} M{M}")


@pytest.mark.parametrize("xdt,sdt", [(torch.float32, torch.bfloat16), (torch.float16, torch.float16),
                                     (torch.bfloat16, torch.float16)])
def test_planned_qmv_dtypes(O, rq, dev, xdt, sdt):
    say(f"planned qmv x={xdt} s={sdt}")
    plan, refs, _, _ = _planned(O, rq, dev, PLAN_SHAPES, 3, 64, 4, 5900, xdt, sdt)
    for y, ref in zip(plan.run(), refs):
        rel_check(y, ref, what=f"planned {xdt} {sdt}")


# The wide kernel (4 < m <= 16, 4- and 8-bit codes): x staged in chunks of
# 1024 columns, so contractions of one partial chunk (512), whole chunks
# (1024, 2048, 8192) and a partial last chunk (1536) are all covered; row
# counts that end mid-block; m = 5 and 9 leave zero A rows in the ring.
WIDE_SHAPES = [(100, 512), (64, 1024), (17, 2048), (40, 1536), (33, 8192)]


@pytest.mark.parametrize("M", [5, 8, 9, 16])
@pytest.mark.parametrize("gs", GROUPS)
@pytest.mark.parametrize("bits", [4, 8])
def test_planned_wide_qmv_parity(O, rq, dev, bits, gs, M):
    say(f"planned wide qmv bits={bits} gs={gs} M={M}")
    plan, refs, _, _ = _planned(O, rq, dev, WIDE_SHAPES, M, gs, bits, 5300 + 10 * bits + gs + M)
    for y, ref in zip(plan.run(), refs):
        rel_check(y, ref, what=f"planned wide b{bits} g{gs} M{M}")


@pytest.mark.parametrize("xdt,sdt", [(torch.float32, torch.bfloat16), (torch.float16, torch.float16),
                                     (torch.bfloat16, torch.float16)])
def test_planned_wide_qmv_dtypes(O, rq, dev, xdt, sdt):
    say(f"planned wide qmv x={xdt} s={sdt}")
    plan, refs, _, _ = _planned(O, rq, dev, WIDE_SHAPES, 8, 64, 4, 5950, xdt, sdt)
    for y, ref in zip(plan.run(), refs):
        rel_check(y, ref, what=f"planned wide {xdt} {sdt}")


# At m <= 8 the wide kernel stages x by pairs of 1024-column chunks and
# restages the next pair behind two barriers: rows of one pair, of a pair and
# a partial chunk (2560, 3584) and of four pairs (8192) in one launch.
WIDE_PAIR_SHAPES = [(100, 512), (17, 2048), (40, 1536), (24, 2560), (20, 3584), (33, 8192)]


@pytest.mark.parametrize("M", [5, 8])
@pytest.mark.parametrize("gs", GROUPS)
@pytest.mark.parametrize("bits", [4, 8])
def test_planned_wide_pair_restaging(O, rq, dev, bits, gs, M):
    """Against the oracle, and bit for bit against each problem run alone
    (a launch's problems do not interact through the restaged ring)."""
    say(f"planned wide pair restaging bits={bits} gs={gs} M={M}")
    seed = 5600 + 10 * bits + gs + M
    plan, refs, xs, ws = _planned(O, rq, dev, WIDE_PAIR_SHAPES, M, gs, bits, seed)
    ys = [y.clone() for y in plan.run()]
    for (R, K), y, ref in zip(WIDE_PAIR_SHAPES, ys, refs):
        rel_check(y, ref, what=f"planned wide pairs b{bits} g{gs} M{M} [{R},{K}]")
    for i, (x, w) in enumerate(zip(xs, ws)):
        alone = rq.GroupedQmv([x], [w], gs, bits, planned=True).run()[0]
        assert bits_equal(ys[i], alone), f"problem {i}: differs from the same problem run alone"


@pytest.mark.parametrize("xdt", [torch.float32, torch.float16])
def test_planned_wide_pair_restaging_dtypes(O, rq, dev, xdt):
    say(f"planned wide pair restaging x={xdt}")
    plan, refs, _, _ = _planned(O, rq, dev, WIDE_PAIR_SHAPES, 6, 64, 4, 5990, xdt, torch.float16)
    for y, ref in zip(plan.run(), refs):
        rel_check(y, ref, what=f"planned wide pairs {xdt}")


def test_planned_rejects_uncovered_sets(O, rq, dev):
    """cols not a multiple of 512, or 4 < m <= 16 with codes other than 4- or
    8-bit: planned=True raises, auto falls back."""
    from rwkvq._lib import RwkvqError
    w = weights(64, 768, 1)
    wq, s, b = (t.to(dev) for t in O.quantize(w, 64, 4))
    x = acts(1, 768, 1).to(dev)
    with pytest.raises(RwkvqError):
        rq.GroupedQmv([x], [(wq, s, b)], 64, 4, planned=True)
    assert rq.GroupedQmv([x], [(wq, s, b)], 64, 4).plan is None
    w = weights(64, 1024, 2)
    wq, s, b = (t.to(dev) for t in O.quantize(w, 64, 3))
    x = acts(8, 1024, 2).to(dev)
    with pytest.raises(RwkvqError):
        rq.GroupedQmv([x], [(wq, s, b)], 64, 3, planned=True)
    assert rq.GroupedQmv([x], [(wq, s, b)], 64, 3).plan is None


def test_planned_many_problems_one_launch(O, rq, dev):
    """150 problems of three contraction sizes (> RQ_MAX_GROUPED): one launch,
    blocks ordered longest first; run twice with new activations in place."""
    shapes = [(64 + 16 * (i % 5), (512, 1024, 2048)[i % 3]) for i in range(150)]
    say("planned qmv, 150 problems")
    plan, refs, xs, ws = _planned(O, rq, dev, shapes, 1, 64, 4, 6000)
    for y, ref in zip(plan.run(), refs):
        rel_check(y, ref, what="planned150")
    # new activations in the same buffers, same plan
    for i, x in enumerate(xs):
        x.copy_(acts(1, x.shape[-1], 7000 + i).to(dev))
    for i, y in enumerate(plan.run()):
        wq, s, b = (t.cpu() for t in ws[i])
        ref = O.quantized_matmul(xs[i].cpu(), wq, s, b, True, 64, 4, out_dtype=torch.float32, weights="exact")
        rel_check(y, ref, what=f"planned150 rerun {i}")


@pytest.mark.parametrize("M", [1, 4, 8, 16])
@pytest.mark.parametrize("bits", [3, 4, 8])
def test_streamed_single_launch_path(O, rq, dev, bits, M):
    """A single problem big enough (>= 2048 16-row blocks) for the streamed
    kernel through rq_qmm itself (3-bit: codes straddling words, the
    mixed-offset pair extraction; M > 4 at 4 and 8 bits: the wide kernel)."""
    R, K = 32768 + 40, 1024
    w = weights(R, K, 8100 + bits)
    wq, s, b = O.quantize(w, 64, bits)
    x = acts(M, K, 8100)
    say(f"streamed single bits={bits} M={M}")
    y = rq.quantized_matmul(x.to(dev), wq.to(dev), s.to(dev), b.to(dev), True, 64, bits)
    rel_check(y, O.quantized_matmul(x, wq, s, b, True, 64, bits, out_dtype=torch.float32, weights="exact"))


@pytest.mark.parametrize("M", [1, 8])
def test_decode_launches_in_a_hip_graph(O, rq, dev, M):
    """A decode step of per-projection launches (rq_qmm_grouped's K-split
    kernel) plus one planned launch, captured once in a HIP graph: every
    replay -- with new activations written in place and eager work between
    replays -- matches the eager launches bit for bit, and the oracle."""
    shapes = [(256, 1024), (512, 2048), (2048, 512)]
    xs, ws = [], []
    for i, (R, K) in enumerate(shapes):
        wq, s, b = O.quantize(weights(R, K, 9100 + i), 64, 4)
        ws.append((wq.to(dev), s.to(dev), b.to(dev)))
        xs.append(acts(M, K, 9100 + i).to(dev))
    singles = [rq.GroupedQmv([x], [w], 64, 4) for x, w in zip(xs, ws)]
    assert all(g.plan is None for g in singles)
    planned = rq.GroupedQmv(xs, ws, 64, 4, planned=True)
    outs = [o for g in singles + [planned] for o in g.outs]

    def step():
        for g in singles + [planned]:
            g.run()

    step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for rep in range(3):
        say(f"hip graph M={M} replay {rep}")
        for i, x in enumerate(xs):
            x.copy_(acts(M, x.shape[-1], 9200 + 10 * rep + i).to(dev))
        step()
        torch.cuda.synchronize()
        eager = [o.clone() for o in outs]
        for o in outs:
            o.zero_()
        graph.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert bits_equal(o, e), f"replay {rep} differs from the eager launches"
        for i, (x, (wq, s, b)) in enumerate(zip(xs, ws)):
            ref = O.quantized_matmul(x.cpu(), wq.cpu(), s.cpu(), b.cpu(), True, 64, 4,
                                     out_dtype=torch.float32, weights="exact")
            rel_check(outs[i], ref, what=f"graph replay {rep} problem {i}")


@pytest.mark.parametrize("rank", [16, 32, 48, 64])
def test_lora_down_matches_fp32(rq, dev, rank):
    """rq_lora_down (z = x . a^T, the QLoRA layer's rank products) against an
    fp32 product of the same bf16 operands: rows ending mid-tile, contractions
    of one k-step to 256, a wave's k-steps past the end (K = 96)."""
    for M, K in [(1, 32), (17, 96), (300, 2048), (4096, 2048), (513, 8192)]:
        g = torch.Generator().manual_seed(M * 7 + K + rank)
        x = torch.randn(M, K, generator=g).to(torch.bfloat16)
        a = (torch.randn(rank, K, generator=g) / K ** 0.5).to(torch.bfloat16)
        say(f"lora_down M={M} K={K} rank={rank}")
        z = rq.lora_down(x.to(dev), a.to(dev))
        assert z.dtype == torch.bfloat16 and tuple(z.shape) == (M, rank)
        ref = x.float() @ a.float().t()
        rel_check(z, ref, what=f"lora_down {M}x{K} r{rank}")


# ---------------------------------------------- autograd / modules / LoRA

def test_autograd_dx_is_transposed_qmm(O, rq, dev):
    R, K, M = 256, 512, 24
    w = weights(R, K, 44)
    wq, s, b = O.quantize(w, 64, 4)
    x = acts(M, K, 44).to(dev).requires_grad_(True)
    say("autograd")
    y = rq.quantized_matmul(x, wq.to(dev), s.to(dev), b.to(dev), True, 64, 4)
    g = acts(M, R, 45)
    y.backward(g.to(dev))
    ref = O.quantized_matmul(g, wq, s, b, False, 64, 4, out_dtype=torch.float32, weights="exact")
    rel_check(x.grad, ref, what="dX")


def test_direct_calls_equal_registered_ops(rq, dev):
    """Eager calls on plain GPU tensors without autograd skip the torch.library
    dispatcher; they must give what the registered ops give, bit for bit, and
    calls that need the dispatcher (autograd, no_grad aside) must still take it."""
    from rwkvq import ops
    R, K, M = 192, 512, 5
    w = weights(R, K, 46).to(dev)
    x = acts(M, K, 46).to(dev)
    assert ops._direct(w, x)
    say("direct vs registered ops")
    got = rq.quantize(w, 64, 4)
    want = torch.ops.rwkvq.quantize(w, 64, 4)
    assert all(bits_equal(a, b) for a, b in zip(got, want))
    wq, s, b = got
    assert bits_equal(rq.dequantize(wq, s, b, 64, 4), torch.ops.rwkvq.dequantize(wq, s, b, 64, 4))
    for tr, xx in ((True, x), (False, acts(M, R, 47).to(dev))):
        assert bits_equal(rq.quantized_matmul(xx, wq, s, b, tr, 64, 4),
                          torch.ops.rwkvq.quantized_matmul(xx, wq, s, b, tr, 64, 4))
    idx = torch.tensor([[3, 0], [191, 7]], device=dev)
    assert bits_equal(rq.quantized_embedding(idx, wq, s, b, 64, 4),
                      torch.ops.rwkvq.quantized_embedding(idx, wq, s, b, 64, 4))
    codes = rq.unpack_codes(wq, 4)
    assert bits_equal(codes, torch.ops.rwkvq.unpack_codes(wq, 4))
    assert bits_equal(rq.pack_codes(codes, 4), torch.ops.rwkvq.pack_codes(codes, 4))
    xg = x.clone().requires_grad_(True)
    assert not ops._direct(xg, wq)
    with torch.no_grad():
        assert ops._direct(xg, wq)
    y = rq.quantized_matmul(xg, wq, s, b, True, 64, 4)
    assert y.grad_fn is not None and bits_equal(y, rq.quantized_matmul(x, wq, s, b, True, 64, 4))


@pytest.mark.parametrize("M", [96, 320])
def test_qlora_layer_forward_backward(rq, dev, M):
    """benchmark config 4 math at a reduced shape: y = qmm(x,Wq) + (a/r)(xA^T)B^T;
    grads of x, A, B against an fp32 dense reference on the dequantized base.
    M=320 runs the fused low-rank term (forward and dX GEMMs), M=96 the
    composed ops."""
    torch.manual_seed(0)
    D, R, r, alpha = 512, 768, 16, 16.0
    lin = torch.nn.Linear(D, R, bias=False).to(dev, torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(weights(R, D, 7).to(dev))
    layer = rq.LoRALinear(lin, rank=r, alpha=alpha, quantize_base=4, q_group_size=64)
    g = torch.Generator().manual_seed(600)
    with torch.no_grad():
        layer.lora_a.copy_((torch.randn(r, D, generator=g) / D ** 0.5).to(torch.bfloat16))
        layer.lora_b.copy_((torch.randn(R, r, generator=g) * 0.01).to(torch.bfloat16))
    x = acts(M, D, 9).to(dev).reshape(M // 16, 16, D).requires_grad_(True)
    say(f"qlora layer M={M}")
    y = layer(x)
    assert y.shape == (M // 16, 16, R)
    dy = acts(M, R, 800).to(dev).reshape(M // 16, 16, R)
    y.backward(dy)
    wd = layer.linear.dequantized_weight().float()
    xr = x.detach().float().requires_grad_(True)
    A = layer.lora_a.detach().float().requires_grad_(True)
    B = layer.lora_b.detach().float().requires_grad_(True)
    yr = xr @ wd.t() + (alpha / r) * ((xr @ A.t()) @ B.t())
    yr.backward(dy.float())
    rel_check(y, yr, what="qlora y")
    rel_check(x.grad, xr.grad, what="qlora dx")
    rel_check(layer.lora_a.grad, A.grad, what="qlora dA")
    rel_check(layer.lora_b.grad, B.grad, what="qlora dB")


def test_quantized_embedding_and_linear_module(O, rq, dev):
    emb = torch.nn.Embedding(1000, 256).to(dev, torch.bfloat16)
    with torch.no_grad():
        emb.weight.copy_(weights(1000, 256, 3).to(dev))
    qe = rq.QuantizedEmbedding.from_embedding(emb, 64, 4)
    idx = torch.tensor([[0, 5, 999], [17, 17, 3]], device=dev)
    say("quantized embedding")
    out = qe(idx)
    owq, os_, ob = O.quantize(weights(1000, 256, 3), 64, 4)
    ref = O.dequantize(owq, os_, ob, 64, 4)[idx.cpu()]
    assert bits_equal(out, ref)
    lin = torch.nn.Linear(256, 96, bias=True).to(dev, torch.bfloat16)
    ql = rq.QuantizedLinear.from_linear(lin, 64, 4)
    x = acts(4, 256, 1).to(dev)
    ref = x.float() @ ql.dequantized_weight().float().t() + lin.bias.float()
    rel_check(ql(x), ref, what="QuantizedLinear")


@pytest.mark.parametrize("bits,gs,sdt", [(4, 64, torch.bfloat16), (3, 32, torch.float16),
                                         (8, 128, torch.float32), (6, 64, torch.bfloat16)])
def test_embedding_gather_dequant(O, rq, dev, bits, gs, sdt):
    """rq_embedding (fused gather + dequantize) is bit-exact to the oracle's
    dequantize of the gathered rows, for int32/int64 indices of any shape,
    repeated indices, and gives NaN rows (not a fault) for indices outside
    the table."""
    R, K = 333, 4 * gs
    w = weights(R, K, 61 + bits, dtype=sdt)
    wq, s, b = O.quantize(w, gs, bits)
    table = O.dequantize(wq, s, b, gs, bits)
    g = torch.Generator().manual_seed(bits)
    idx = torch.randint(0, R, (3, 7, 5), generator=g)
    idx[0, 0, 0], idx[2, 6, 4] = 0, R - 1
    say(f"embedding bits={bits} gs={gs} sdt={sdt}")
    for it in (torch.int64, torch.int32):
        out = rq.quantized_embedding(idx.to(dev, it), wq.to(dev), s.to(dev), b.to(dev), gs, bits)
        assert out.shape == (3, 7, 5, K) and out.dtype == sdt
        assert bits_equal(out, table[idx])
    bad = torch.tensor([5, -1, R, 7], device=dev)
    out = rq.quantized_embedding(bad, wq.to(dev), s.to(dev), b.to(dev), gs, bits).cpu()
    assert bits_equal(out[0], table[5]) and bits_equal(out[3], table[7])
    assert torch.isnan(out[1].float()).all() and torch.isnan(out[2].float()).all()
    empty = rq.quantized_embedding(torch.zeros(0, dtype=torch.int64, device=dev), wq.to(dev),
                                   s.to(dev), b.to(dev), gs, bits)
    assert empty.shape == (0, K)


# --------------------------------------------------- determinism / edges

def test_repeated_launches_bitwise_identical(rq, dev):
    """Race regression: five launches of each kernel family give identical bits."""
    w = weights(4096, 2048, 12).to(dev)
    wq, s, b = rq.quantize(w, 64, 4)
    say("determinism")
    for M, tr in ((1, True), (8, True), (256, True), (256, False)):
        x = acts(M, 2048 if tr else 4096, M).to(dev)
        outs = [rq.quantized_matmul(x, wq, s, b, tr, 64, 4) for _ in range(5)]
        assert all(torch.equal(outs[0], o) for o in outs[1:]), (M, tr)
    q2 = [rq.quantize(w, 64, 4)[0] for _ in range(3)]
    assert all(torch.equal(q2[0], q) for q in q2)


def test_empty_and_unaligned_inputs(O, rq, dev):
    w = weights(64, 256, 1)
    wq, s, b = O.quantize(w, 64, 4)
    wq, s, b = wq.to(dev), s.to(dev), b.to(dev)
    say("empty/unaligned")
    y = rq.quantized_matmul(torch.empty(0, 256, device=dev, dtype=torch.bfloat16), wq, s, b,
                            True, 64, 4)
    assert y.shape == (0, 64)
    big = acts(3, 257, 2).to(dev)
    x = big[:, 1:]                      # storage offset 1 element: not 16-byte aligned
    y = rq.quantized_matmul(x, wq, s, b, True, 64, 4)
    ref = O.quantized_matmul(x.cpu().contiguous(), wq.cpu(), s.cpu(), b.cpu(), True, 64, 4,
                             out_dtype=torch.float32, weights="exact")
    rel_check(y, ref, what="unaligned x")
    xt = acts(256, 3, 4).to(dev).t()    # non-contiguous view
    y = rq.quantized_matmul(xt, wq, s, b, True, 64, 4)
    ref = O.quantized_matmul(xt.cpu().contiguous(), wq.cpu(), s.cpu(), b.cpu(), True, 64, 4,
                             out_dtype=torch.float32, weights="exact")
    rel_check(y, ref, what="transposed view x")


def test_uint32_words_accepted(O, rq, dev):
    w = weights(32, 128, 2)
    wq, s, b = O.quantize(w, 64, 4)
    x = acts(1, 128, 2)
    y1 = rq.quantized_matmul(x.to(dev), wq.to(dev).view(torch.uint32), s.to(dev), b.to(dev))
    y2 = rq.quantized_matmul(x.to(dev), wq.to(dev), s.to(dev), b.to(dev))
    assert torch.equal(y1, y2)


@pytest.mark.parametrize("transpose", [True, False])
def test_bound_qmm_matches_op(O, rq, dev, transpose):
    """BoundQmm.run() is the same rq_qmm call as quantized_matmul, on a fixed
    output buffer; rewriting x in place between runs changes the result."""
    gs, bits, R, K, M = 64, 4, 192, 1024, 260
    w = weights(R, K, 41)
    wq, s, b = (t.to(dev) for t in O.quantize(w, gs, bits))
    x = acts(M, K if transpose else R, 43).to(dev)
    bound = rq.BoundQmm(x, wq, s, b, transpose, gs, bits)
    y1 = bound.run().clone()
    assert torch.equal(y1, rq.quantized_matmul(x, wq, s, b, transpose, gs, bits))
    x.copy_(acts(M, x.shape[1], 47).to(dev))
    y2 = bound.run()
    assert y2.data_ptr() == bound.out.data_ptr()
    assert torch.equal(y2, rq.quantized_matmul(x, wq, s, b, transpose, gs, bits))
    assert not torch.equal(y1, y2)
    with pytest.raises(ValueError):
        rq.BoundQmm(x, wq, s, b, transpose, gs, bits, out=torch.empty(1, device=dev))


QUANT_TARGETS = ("emb", "head") + tuple(f"blocks.{i}.cmix.{n}" for i in range(2)
                                          for n in ("key", "value"))


def _check_quantized_module(O, mod, w_src, gs, bits, what):
    """mod's packed words, scales and biases equal O.quantize of the source
    weight bit for bit."""
    owq, os_, ob = O.quantize(w_src, gs, bits)
    assert mod.bits == bits and mod.group_size == gs, what
    assert bits_equal(mod.weight, owq), f"{what}: packed words"
    assert bits_equal(mod.scales, os_), f"{what}: scales"
    assert bits_equal(mod.biases, ob), f"{what}: biases"
    return owq, os_, ob


def _check_products(O, model, idx, packed, what):
    """Every quantized module's HIP output against the oracle on the packed
    tensors: the embedding rows bit-exact to O.dequantize, the linear products
    within rel-err 1e-2 of O.quantized_matmul over the same bf16 inputs."""
    parts = model.forward_parts(idx)
    inputs = {"head": parts["emb"]}
    for i in range(len(model.blocks)):
        inputs[f"blocks.{i}.cmix.key"] = parts["emb"]
        inputs[f"blocks.{i}.cmix.value"] = parts[f"blocks.{i}.cmix.key"]
    wq, s, b, gs, bits = packed["emb"]
    rows = O.dequantize(wq, s, b, gs, bits)[idx.cpu().reshape(-1)].reshape(parts["emb"].shape)
    assert bits_equal(parts["emb"], rows), f"{what}: embedding rows"
    for path, x in inputs.items():
        wq, s, b, gs, bits = packed[path]
        ref = O.quantized_matmul(x.cpu(), wq, s, b, True, gs, bits, out_dtype=torch.float32,
                                 weights="exact")
        rel_check(parts[path], ref, what=f"{what}: {path}")


def test_quantize_base_model_gpu_bit_exact(O, rq, dev):
    """quantize_base_model (rwkv_metal/lora/finetune.py:70-91) on a CUDA model
    with the reference's module layout: exactly BIG_QUANT_TARGETS (cmix.key,
    cmix.value, head, emb; finetune.py:42) are swapped, each swapped module's
    (weight, scales, biases) is bit-exact to O.quantize of the original weight,
    the tmix projections and the low-rank branch keep their float weights, and
    the swapped modules' outputs match the oracle's products."""
    from rwkv_layout import Tiny
    m = Tiny(d=256, n=2, vocab=512, device=dev, seed=71)
    src = {k: v.detach().cpu().clone() for k, v in m.state_dict().items()}
    say("quantize_base_model bits=4 gs=64")
    assert rq.quantize_base_model(m, bits=4, group_size=64) is m
    packed = {}
    for path, mod in m.named_modules():
        if isinstance(mod, (rq.QuantizedLinear, rq.QuantizedEmbedding)):
            assert path in QUANT_TARGETS, f"{path} quantized but not a target"
            assert isinstance(mod, rq.QuantizedEmbedding) == (path == "emb"), path
            packed[path] = (*_check_quantized_module(O, mod, src[f"{path}.weight"], 64, 4, path),
                            64, 4)
    assert sorted(packed) == sorted(QUANT_TARGETS)
    for i, blk in enumerate(m.blocks):
        for name in ("r_proj", "k_proj", "v_proj", "o_proj", "w_lora"):
            lin = getattr(blk.tmix, name)
            assert type(lin) is torch.nn.Linear, f"blocks.{i}.tmix.{name} was swapped"
            assert bits_equal(lin.weight, src[f"blocks.{i}.tmix.{name}.weight"])
    idx = torch.tensor([[0, 5, 77, 511], [3, 3, 200, 1]], device=dev)
    _check_products(O, m, idx, packed, "quantize_base_model")


def test_quantized_checkpoint_against_oracle(O, rq, dev, tmp_path):
    """save_quantized / load_quantized (the packed checkpoint of an nn.quantize'd
    model, keys <path>.weight/.scales/.biases as MLX saves them;
    rwkv_metal/model/convert.py:437, rwkv_metal/lora/lora.py:140-148) with a
    3-bit body and an 8-bit head chosen per module: the file's tensors are
    O.quantize of the source weights bit for bit, the loaded model gets the
    same bits and group sizes back from the stored shapes, and its HIP outputs
    match the oracle's products of the file's tensors."""
    from safetensors.torch import load_file
    from rwkv_layout import Tiny
    from rwkvq import io as rio

    src_model = Tiny(d=256, n=2, vocab=512, device=dev, seed=73)
    src = {k: v.detach().cpu().clone() for k, v in src_model.state_dict().items()}
    setting = {p: (64, 8 if p == "head" else 3) for p in QUANT_TARGETS}
    say("checkpoint: quantize 3-bit body / 8-bit head, save, load")
    rq.quantize_model(src_model, 64, 3, class_predicate=lambda p, mod: (
        {"bits": 8} if p == "head" else p in QUANT_TARGETS))
    path = str(tmp_path / "m.safetensors")
    rio.save_quantized(src_model, path)
    assert rio.quantization_config(path) == {"group_size": 64, "bits": 3,
                                             "head": {"group_size": 64, "bits": 8}}
    f = load_file(path)
    packed = {}
    for p, (gs, bits) in setting.items():
        owq, os_, ob = O.quantize(src[f"{p}.weight"], gs, bits)
        assert f[f"{p}.weight"].dtype == torch.uint32, p
        assert torch.equal(f[f"{p}.weight"].view(torch.int32), owq), f"{p}: file words"
        assert bits_equal(f[f"{p}.scales"], os_) and bits_equal(f[f"{p}.biases"], ob), p
        packed[p] = (f[f"{p}.weight"].view(torch.int32), f[f"{p}.scales"], f[f"{p}.biases"],
                     gs, bits)
    for k, v in src.items():        # every float tensor is stored as it was
        if k.rpartition(".")[0] not in setting:
            assert bits_equal(f[k], v), k

    dst = Tiny(d=256, n=2, vocab=512, device=dev, seed=999)   # different float weights
    rio.load_quantized(dst, path)
    for p, (gs, bits) in setting.items():
        mod = dst.get_submodule(p)
        assert (mod.group_size, mod.bits) == (gs, bits), p
        assert bits_equal(mod.weight, packed[p][0]), p
    for i in range(2):              # unquantized modules took the file's weights
        assert bits_equal(dst.blocks[i].tmix.r_proj.weight, src[f"blocks.{i}.tmix.r_proj.weight"])
    idx = torch.tensor([[1, 7, 511, 0]], device=dev)
    _check_products(O, dst, idx, packed, "loaded checkpoint")


# ------------------------------------------------------------ sb6 / K3

@pytest.mark.parametrize("xbits", [0, 1, 2])
def test_sb6_dequantize_and_repack_bit_exact(O, rq, dev, xbits):
    """rq_sb6_dequantize (fp32 and bf16) and rq_sb6_to_affine (packed codes,
    clamped fp32 scales, biases; scales-only mode) against the oracle, bit for
    bit, including subnormal float16 super-block scales."""
    import sb6_k3 as k3
    from rwkvq import sb6
    R, K, gw_sb = 37, 1024, 8
    codes, qs, qm, d, dm = k3.random_sb6(R, K, xbits, gw_sb, seed=100 + xbits, tiny=True)
    qblk, qsqm, ddm = k3.encode(codes, qs, qm, d, dm, xbits)
    say(f"sb6 xbits={xbits}")
    lin = rq.RwkvqLinear(qblk.to(dev), qsqm.to(dev), ddm.to(dev), (R, K), 32, gw_sb, xbits)
    want = O.sb6_dequantize(qblk, qsqm, ddm, R, K, gw_sb, xbits)
    assert bits_equal(lin._dequant_w_fp32(), want)
    assert bits_equal(lin._dequant_w(), want.to(torch.bfloat16))
    wq, sc, bi = sb6._to_affine(lin)
    assert torch.equal(wq.cpu(), O.pack(O.sb6_codes(qblk, R, K, xbits), 4 + xbits))
    osc, omn = O.sb6_scale_min(qsqm, ddm, R, K, gw_sb, clamp=True)
    assert bits_equal(sc, osc) and bits_equal(bi, omn)
    hyb = rq.RwkvqHybridLinear(lin)
    hs, hb = hyb._expand_scale_bias()
    assert bits_equal(hs, osc) and bits_equal(hb, omn) and torch.equal(hyb.wq, wq)


@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
def test_sb6_linear_modules(O, rq, dev, xdt):
    """The three sb6 bases agree with the oracle's products: RwkvqNativeLinear
    and RwkvqHybridLinear (quantized_matmul on the repacked layout, fp32 x,
    group 32; identical bits to each other) and RwkvqLinear (dense dequant +
    matmul), within rel-err 1e-2, at decode (M=1, 8) and prefill (M=300)."""
    import sb6_k3 as k3
    R, K, gw_sb, xbits = 256, 2048, 8, 2
    codes, qs, qm, d, dm = k3.random_sb6(R, K, xbits, gw_sb, seed=7)
    qs[qs == 0] = 1
    qblk, qsqm, ddm = k3.encode(codes, qs, qm, d, dm, xbits)
    lin = rq.RwkvqLinear(qblk.to(dev), qsqm.to(dev), ddm.to(dev), (R, K), 32, gw_sb, xbits)
    nat, hyb = rq.RwkvqNativeLinear(lin), rq.RwkvqHybridLinear(lin)
    wq = O.pack(O.sb6_codes(qblk, R, K, xbits), 4 + xbits)
    osc, omn = O.sb6_scale_min(qsqm, ddm, R, K, gw_sb, clamp=True)
    dense = O.sb6_dequantize(qblk, qsqm, ddm, R, K, gw_sb, xbits).double()
    for M in (1, 8, 300):
        x = acts(M, K, M, xdt)
        say(f"sb6 modules x={xdt} M={M}")
        yn = nat(x.to(dev))
        assert yn.dtype == xdt and torch.equal(yn, hyb(x.to(dev)))
        ref = O.quantized_matmul(x.float(), wq, osc, omn, True, 32, 6, out_dtype=torch.float32,
                                 weights="exact")
        rel_check(yn, ref, what=f"native M{M}")
        yl = lin(x.to(dev))
        rel_check(yl, x.double() @ dense.t(), what=f"RwkvqLinear M{M}")


def test_add_lora_rwkvq_from_sidecar(O, rq, dev, tmp_path):
    """add_lora_rwkvq swaps tmix projections (LoRA-wrapped), cmix key/value and
    the head for the sb6 base read from a sidecar (<path>.safetensors +
    <path>.json, official key names); only the adapters train; the forward of
    a wrapped projection equals the base plus the LoRA term."""
    import json
    from safetensors.torch import save_file
    from torch import nn
    import sb6_k3 as k3

    D, V, L = 256, 512, 2

    class TMix(nn.Module):
        def __init__(self):
            super().__init__()
            for n in ("r_proj", "k_proj", "v_proj", "o_proj"):
                setattr(self, n, nn.Linear(D, D, bias=False))

    class CMix(nn.Module):
        def __init__(self):
            super().__init__()
            self.key, self.value = nn.Linear(D, 4 * D, bias=False), nn.Linear(4 * D, D, bias=False)

    class Blk(nn.Module):
        def __init__(self):
            super().__init__()
            self.tmix, self.cmix = TMix(), CMix()

    class Model(nn.Module):
        def __init__(self):
            super().__init__()
            self.blocks = nn.ModuleList([Blk() for _ in range(L)])
            self.head = nn.Linear(D, V, bias=False)

    shapes = {"head.weight": (V, D)}
    for i in range(L):
        for n in ("receptance", "key", "value", "output"):
            shapes[f"blocks.{i}.att.{n}.weight"] = (D, D)
        shapes[f"blocks.{i}.ffn.key.weight"] = (4 * D, D)
        shapes[f"blocks.{i}.ffn.value.weight"] = (D, 4 * D)
    arrays, meta = {}, {"tensors": {}}
    for j, (key, (R, K)) in enumerate(shapes.items()):
        xb = j % 3
        codes, qs, qm, d, dm = k3.random_sb6(R, K, xb, 4, seed=j)
        qblk, qsqm, ddm = k3.encode(codes, qs, qm, d, dm, xb)
        arrays[f"{key}::qblk"], arrays[f"{key}::qsqm"], arrays[f"{key}::ddm"] = qblk, qsqm, ddm
        meta["tensors"][key] = {"kind": "sb6", "shape": [R, K], "gw_gs": 32, "gw_sb": 4,
                                "xbits": xb}
    side = str(tmp_path / "model.rwkvq_mlx")
    save_file(arrays, side + ".safetensors")
    with open(side + ".json", "w") as f:
        json.dump(meta, f)

    model = Model().to(dev, torch.bfloat16)
    model, info = rq.add_lora_rwkvq(model, side, rank=8, alpha=16.0, layers=[-1])
    say("add_lora_rwkvq")
    assert info["num_lora_adapters"] == 4 and info["wrapped_per_block"] == [
        "tmix.k_proj", "tmix.o_proj", "tmix.r_proj", "tmix.v_proj"]
    blk = model.blocks[1]
    assert isinstance(blk.tmix.r_proj, rq.LoRALinear)
    assert isinstance(blk.tmix.r_proj.linear, rq.RwkvqNativeLinear)
    assert isinstance(blk.cmix.value, rq.RwkvqNativeLinear) and blk.cmix.value.bits == 4 + (
        list(shapes).index("blocks.1.ffn.value.weight") % 3)
    assert isinstance(model.head, rq.RwkvqNativeLinear)
    assert isinstance(model.blocks[0].tmix.r_proj, nn.Linear)   # layer 0 not selected
    trainable = {n for n, p in model.named_parameters() if p.requires_grad}
    assert trainable == {f"blocks.1.tmix.{n}.lora_{ab}" for n in ("r_proj", "k_proj", "v_proj",
                                                                   "o_proj") for ab in "ab"}
    with torch.no_grad():
        blk.tmix.k_proj.lora_b.normal_()
    x = acts(4, D, 3).to(dev)
    lay = blk.tmix.k_proj
    y = lay(x)
    ref = lay.linear(x).float() + lay.scale * ((x.float() @ lay.lora_a.float().t())
                                               @ lay.lora_b.float().t())
    rel_check(y, ref, what="lora over sb6")
    with pytest.raises(NotImplementedError):
        rq.load_sidecar(str(tmp_path / "model.rwkvq"))


@pytest.mark.parametrize("transpose,rank", [(True, 16), (True, 32), (True, 64), (False, 16),
                                            (False, 48)])
def test_qmm_lora_fused_term(O, rq, dev, transpose, rank):
    """rq_qmm_lora: the low-rank term scale * z L^T added in the 64-wide-stage
    GEMMs' output stage, against the oracle product plus the term in float64
    (partial tiles in both dims); a problem outside those kernels (M=64)
    returns RQ_EUNSUPPORTED internally and the op composes the same result."""
    from rwkvq import ops
    gs, bits, R, K = 64, 4, 320, 1024
    w = weights(R, K, 71 + rank)
    wq, s, b = O.quantize(w, gs, bits)
    n_in, n_out = (K, R) if transpose else (R, K)
    g = torch.Generator().manual_seed(rank)
    L = (torch.randn(n_out, rank, generator=g) * 0.05).to(torch.bfloat16)
    for M in (300, 64):
        x = acts(M, n_in, M + rank)
        z = (torch.randn(M, rank, generator=g)).to(torch.bfloat16)
        say(f"qmm_lora transpose={transpose} rank={rank} M={M}")
        args = [t.to(dev) for t in (x, wq, s, b, z, L)]
        fused = ops._qmm_lora_fused(*args, 2.0, transpose, gs, bits)
        assert (fused is not None) == (M == 300)
        y = rq.quantized_matmul_lora(*args, 2.0, transpose, gs, bits)
        ref = O.quantized_matmul(x, wq, s, b, transpose, gs, bits, out_dtype=torch.float32,
                                 weights="exact").double()
        ref = ref + 2.0 * (z.double() @ L.double().t())
        rel_check(y, ref, what=f"qmm_lora t{transpose} r{rank} M{M}")
        if fused is not None:
            rel_check(fused, ref, what="fused")

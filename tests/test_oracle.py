"""Pins the CPU oracle (oracle/rq_oracle.c) before it is trusted as the checker.

Each check is an independent statement of what the reference fixes, not a
retyping of the oracle's formula:
  * packing: a Python big-integer bitstream, hand-derived word/bit positions
    (rwkv_metal/lora/rwkvq_native.py:18-33) and the reference's own one-hot
    probe (tests/dev_reverse_mlx_pack.py:8-44) with hand-derived codes;
  * quantize: nearest-code brute force, exact extremes, exactly representable
    zero, constant and all-zero groups, reconstruction bound;
  * dequantize: torch's own bf16/fp32 elementwise arithmetic (multiply then
    add, each rounded -- MLX's composite op order);
  * quantized_matmul: float64 dense matmul of the dequantized weights and a
    pure-Python loop on tiny shapes, for both transposes.
"""
import math

import numpy as np
import pytest
import torch

BITS = (2, 3, 4, 5, 6, 8)
GROUPS = (32, 64, 128)


def bigint_pack(codes, bits):
    """Row-wise LSB-first bitstream via Python integers."""
    rows, K = codes.shape
    out = np.zeros((rows, K * bits // 32), dtype=np.uint32)
    for r in range(rows):
        acc = 0
        for j in range(K):
            acc |= int(codes[r, j]) << (j * bits)
        for w in range(K * bits // 32):
            out[r, w] = (acc >> (32 * w)) & 0xFFFFFFFF
    return out


@pytest.mark.parametrize("bits", BITS)
def test_pack_matches_bigint_bitstream(O, bits):
    g = torch.Generator().manual_seed(100 + bits)
    codes = torch.randint(0, 1 << bits, (5, 256), generator=g, dtype=torch.int64).to(torch.uint8)
    wq = O.pack(codes, bits)
    ref = bigint_pack(codes.numpy(), bits)
    assert np.array_equal(wq.numpy().view(np.uint32), ref)
    assert torch.equal(O.unpack(wq, bits), codes)


def _one_code(bits, pos, val, K=64):
    c = torch.zeros(1, K, dtype=torch.uint8)
    c[0, pos] = val
    return c


def test_pack_worked_positions(O):
    # 4-bit: word = c0 | c1<<4 | ... | c7<<28
    c = torch.tensor([[0, 1, 2, 3, 4, 5, 6, 7] + [0] * 24], dtype=torch.uint8)
    assert O.pack(c, 4)[0, 0].item() & 0xFFFFFFFF == 0x76543210
    # 8-bit: c0 | c1<<8 | c2<<16 | c3<<24
    c = torch.tensor([[1, 2, 3, 4] + [0] * 28], dtype=torch.uint8)
    assert O.pack(c, 8)[0, 0].item() & 0xFFFFFFFF == 0x04030201
    u = lambda t: [int(v) & 0xFFFFFFFF for v in t[0].tolist()]
    # 3-bit: code 10 = bits 30..32 -> word0 bits 30,31 and word1 bit 0
    assert u(O.pack(_one_code(3, 10, 0b111, 32), 3)) == [0xC0000000, 0x1, 0x0]
    # 3-bit: code 21 = bits 63..65 -> word1 bit 31 (lsb of 0b101) and word2 bits 0..1 (0b10)
    assert u(O.pack(_one_code(3, 21, 0b101, 32), 3)) == [0x0, 0x80000000, 0x2]
    # 6-bit: code 5 = bits 30..35; code 10 = bits 60..65
    assert u(O.pack(_one_code(6, 5, 0x3F, 32), 6))[:2] == [0xC0000000, 0xF]
    assert u(O.pack(_one_code(6, 10, 0x3F, 32), 6))[1:3] == [0xF0000000, 0x3]
    # 5-bit: code 6 = bits 30..34 -> word0 bits 30,31 and word1 bits 0..2
    assert u(O.pack(_one_code(5, 6, 0x1F, 32), 5))[:2] == [0xC0000000, 0x7]


def test_reference_probe_6bit_g32(O):
    """tests/dev_reverse_mlx_pack.py:20-44: anchors 0 and 31 fix min/max, the
    interior holds 15.0; moving one interior position to 20.0 must change only
    the 6 bits of that position.  Hand derivation for this input:
      min=0, max=31, |min|<=|max| -> scale = -(31/63), edge = 31,
      q0 = rint(31/scale) = -63 -> scale = 31/-63, bias = 31;
      code(0) = 63, code(15) = rint(32.516) = 33, code(31) = 0, code(20) = rint(22.35) = 22."""
    base = [0.0] + [15.0] * 30 + [31.0]
    w = torch.tensor([base], dtype=torch.float32)
    wq, s, b = O.quantize(w, group_size=32, bits=6)
    assert s.item() == np.float32(31.0) / np.float32(-63.0)
    assert b.item() == 31.0
    assert O.unpack(wq, 6)[0].tolist() == [63] + [33] * 30 + [0]
    row = lambda t: sum((int(v) & 0xFFFFFFFF) << (32 * i) for i, v in enumerate(t[0].tolist()))
    base_bits = row(wq)
    for p in range(1, 31):
        vals = list(base)
        vals[p] = 20.0
        wq_p, s_p, b_p = O.quantize(torch.tensor([vals]), group_size=32, bits=6)
        assert s_p.item() == s.item() and b_p.item() == b.item()
        diff = row(wq_p) ^ base_bits
        assert diff & ~(0x3F << (6 * p)) == 0, f"position {p} touched bits outside its field"
        assert (row(wq_p) >> (6 * p)) & 0x3F == 22


def _groups_f32(gs, n, seed):
    g = torch.Generator().manual_seed(seed)
    kinds = [
        torch.randn(n, gs, generator=g) * 0.02,
        torch.rand(n, gs, generator=g) * 3 + 0.5,          # all positive
        -(torch.rand(n, gs, generator=g) * 3 + 0.5),       # all negative
        torch.randn(n, gs, generator=g) * torch.logspace(-4, 4, n).unsqueeze(1),
    ]
    w = torch.cat(kinds)
    w[::7, 3] = 0.0   # exact zeros inside groups
    return w


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("gs", GROUPS)
def test_quantize_nearest_code_and_extremes(O, bits, gs):
    n_bins = (1 << bits) - 1
    w = _groups_f32(gs, 16, 7 * bits + gs)
    wq, s, b = O.quantize(w, group_size=gs, bits=bits)   # one group per row, f32 scales
    codes = O.unpack(wq, bits).to(torch.float64)
    s64, b64, w64 = s.double(), b.double(), w.double()
    recon = s64 * codes + b64
    err = (w64 - recon).abs()
    # every code is the nearest grid point (up to fp32 rounding of (w-b)/s)
    grid = s64 * torch.arange(n_bins + 1, dtype=torch.float64) + b64      # [rows, n_bins+1]
    best = (w64.unsqueeze(-1) - grid.unsqueeze(1)).abs().min(-1).values
    assert torch.all(err <= best + 1e-5 * s64.abs() + 1e-12)
    # inside the grid the error is at most half a step (the zero-point rounding
    # can leave the far extreme outside the grid, where the nearest end is used)
    lo, hi = grid.min(-1, keepdim=True).values, grid.max(-1, keepdim=True).values
    inside = (w64 >= lo) & (w64 <= hi)
    assert torch.all(err[inside] <= (s64.abs() * (0.5 + 1e-5) + 1e-12).expand_as(err)[inside])
    # the larger-magnitude extreme is stored exactly as the bias, at code 0
    mn, mx = w.min(1).values, w.max(1).values
    edge = torch.where(mn.abs() > mx.abs(), mn, mx)
    nz = b != 0
    assert torch.equal(b[nz.squeeze(1)].squeeze(1), edge[nz.squeeze(1)])
    idx = torch.where(mn.abs() > mx.abs(), w.argmin(1), w.argmax(1))
    assert torch.all(codes[torch.arange(len(w)), idx][nz.squeeze(1)] == 0)
    # zero is exactly representable: code(0) = -q0 and s*code + b == 0 in exact arithmetic
    rows0 = torch.nonzero((w == 0).any(1) & nz.squeeze(1)).flatten()
    for r in rows0.tolist():
        c = codes[r, (w[r] == 0).nonzero()[0, 0]]
        assert abs(s64[r, 0] * c + b64[r, 0]) <= 4e-7 * abs(b64[r, 0])


@pytest.mark.parametrize("bits", BITS)
def test_quantize_constant_and_zero_groups(O, bits):
    w = torch.tensor([[0.0] * 64, [0.75] * 64, [-3.5] * 64], dtype=torch.bfloat16)
    wq, s, b = O.quantize(w, group_size=64, bits=bits)
    codes = O.unpack(wq, bits)
    assert torch.all(codes == 0)
    assert b.float().tolist() == [[0.0], [0.75], [-3.5]]
    dq = O.dequantize(wq, s, b, 64, bits)
    assert torch.equal(dq, w)


@pytest.mark.parametrize("sdt", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("bits", (3, 4, 8))
def test_dequantize_matches_torch_elementwise(O, sdt, bits):
    g = torch.Generator().manual_seed(3 + bits)
    R, K, gs = 16, 256, 64
    codes = torch.randint(0, 1 << bits, (R, K), generator=g).to(torch.uint8)
    wq = O.pack(codes, bits)
    s = (torch.randn(R, K // gs, generator=g) * 0.01).to(sdt)
    b = (torch.randn(R, K // gs, generator=g) * 0.1).to(sdt)
    got = O.dequantize(wq, s, b, gs, bits)
    s_e = s.repeat_interleave(gs, 1)
    b_e = b.repeat_interleave(gs, 1)
    ref = codes.to(sdt) * s_e      # torch rounds the product to sdt
    ref = ref + b_e                # and the sum again
    assert got.dtype == sdt
    assert torch.equal(got.view(torch.int16) if sdt != torch.float32 else got.view(torch.int32),
                       ref.view(torch.int16) if sdt != torch.float32 else ref.view(torch.int32))


@pytest.mark.parametrize("transpose", [True, False])
@pytest.mark.parametrize("bits,gs", [(4, 64), (3, 64), (8, 32), (5, 128)])
def test_qmm_matches_dense_float64(O, transpose, bits, gs):
    g = torch.Generator().manual_seed(bits * 10 + gs)
    R, K, M = 48, 256, 5
    w = (torch.randn(R, K, generator=g) * 0.02).to(torch.bfloat16)
    wq, s, b = O.quantize(w, gs, bits)
    wd = O.dequantize(wq, s, b, gs, bits).double()
    x = torch.randn(M, K if transpose else R, generator=g).to(torch.bfloat16)
    y = O.quantized_matmul(x, wq, s, b, transpose, gs, bits, out_dtype=torch.float32)
    ref = x.double() @ (wd.t() if transpose else wd)
    assert y.shape == ref.shape
    assert torch.allclose(y.double(), ref, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("transpose", [True, False])
@pytest.mark.parametrize("bits", [3, 4, 8])
def test_qmm_exact_weights_match_dense_float64(O, transpose, bits):
    """weights="exact": s*q + b from the unpacked codes (torch.bitwise
    extraction below, independent of the C code) in float64."""
    g = torch.Generator().manual_seed(300 + bits)
    R, K, M, gs = 40, 256, 3, 64
    w = (torch.randn(R, K, generator=g) * 0.02).to(torch.bfloat16)
    wq, s, b = O.quantize(w, gs, bits)
    words = wq.view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    bitstream = [sum(int(words[r, i]) << (32 * i) for i in range(words.shape[1])) for r in range(R)]
    codes = torch.tensor([[(row >> (k * bits)) & ((1 << bits) - 1) for k in range(K)]
                          for row in bitstream], dtype=torch.float64)
    we = codes * s.double().repeat_interleave(gs, 1) + b.double().repeat_interleave(gs, 1)
    x = torch.randn(M, K if transpose else R, generator=g).to(torch.bfloat16)
    y = O.quantized_matmul(x, wq, s, b, transpose, gs, bits, out_dtype=torch.float32,
                           weights="exact")
    ref = x.double() @ (we.t() if transpose else we)
    assert torch.allclose(y.double(), ref, rtol=1e-6, atol=1e-6)
    # the two weight forms differ only by the bf16 rounding of s*q and +b
    ym = O.quantized_matmul(x, wq, s, b, transpose, gs, bits, out_dtype=torch.float32).double()
    assert ((ym - ref).norm() / ref.norm()).item() < 1.5e-2


def test_qmm_tiny_python_loop(O):
    g = torch.Generator().manual_seed(5)
    R, K, M, gs, bits = 3, 64, 2, 32, 4
    w = torch.randn(R, K, generator=g)
    wq, s, b = O.quantize(w, gs, bits)             # f32 scales
    codes = O.unpack(wq, bits)
    x = torch.randn(M, K, generator=g)
    y = O.quantized_matmul(x, wq, s, b, True, gs, bits)
    for m in range(M):
        for r in range(R):
            acc = 0.0
            for k in range(K):
                sc, bi = float(s[r, k // gs]), float(b[r, k // gs])
                wv = float(np.float32(np.float32(sc * int(codes[r, k])) + np.float32(bi)))
                acc += float(x[m, k]) * wv
            assert math.isclose(float(y[m, r]), acc, rel_tol=1e-6, abs_tol=1e-6)
    x2 = torch.randn(M, R, generator=g)
    y2 = O.quantized_matmul(x2, wq, s, b, False, gs, bits)
    for m in range(M):
        for k in range(K):
            acc = 0.0
            for r in range(R):
                sc, bi = float(s[r, k // gs]), float(b[r, k // gs])
                wv = float(np.float32(np.float32(sc * int(codes[r, k])) + np.float32(bi)))
                acc += float(x2[m, r]) * wv
            assert math.isclose(float(y2[m, k]), acc, rel_tol=1e-6, abs_tol=1e-6)


def test_quantize_rejects_bad_arguments(O):
    w = torch.zeros(2, 64)
    with pytest.raises(ValueError):
        O.quantize(w, 48, 4)
    with pytest.raises(ValueError):
        O.quantize(w, 64, 7)
    with pytest.raises(ValueError):
        O.quantize(torch.zeros(2, 96), 64, 4)


# ------------------------------------------------------------ sb6 / K3

@pytest.mark.parametrize("xbits", [0, 1, 2])
def test_sb6_oracle_matches_the_layout_text(O, xbits):
    """The oracle's sb6 decode against an independent encoder written from
    the layout text (tests/sb6_k3.py): codes round-trip exactly, scale/min are
    numpy's f16(qs*d) / f16(qm*dm), and the dense weight is code*scale + min
    in fp32, bit for bit (including subnormal float16 super-block scales)."""
    import sb6_k3 as k3
    R, K, gw_sb = 7, 512, 4
    codes, qs, qm, d, dm = k3.random_sb6(R, K, xbits, gw_sb, seed=xbits, tiny=True)
    qblk, qsqm, ddm = k3.encode(codes, qs, qm, d, dm, xbits)
    assert torch.equal(O.sb6_codes(qblk, R, K, xbits), torch.from_numpy(codes).to(torch.uint8))
    sc, mn = O.sb6_scale_min(qsqm, ddm, R, K, gw_sb)
    esc, emn = k3.scale_min(qs, qm, d, dm, gw_sb)
    assert np.array_equal(sc.numpy().view(np.int32), esc.view(np.int32))
    assert np.array_equal(mn.numpy().view(np.int32), emn.view(np.int32))
    w = O.sb6_dequantize(qblk, qsqm, ddm, R, K, gw_sb, xbits)
    assert np.array_equal(w.numpy().view(np.int32), k3.dense(codes, qs, qm, d, dm, gw_sb).view(np.int32))


def test_sb6_oracle_hand_worked_block(O):
    """One block decoded by hand: byte 0 = 0xA3 gives code 0 = 3 and code 16
    = 10; bit 0 of the first plane adds 16 to code 0, bit 16 of the second adds
    32 to code 16; qs = 5, d = 0.5 -> scale 2.5; qm = -3 (byte 0xFD), dm = 0.25
    -> min -0.75; w0 = 19*2.5 - 0.75 = 46.75, w16 = 42*2.5 - 0.75 = 104.25."""
    blk = np.zeros(24, dtype=np.uint8)
    blk[0] = 0xA3
    blk[16:20] = np.array([1, 0, 0, 0], dtype=np.uint8)        # plane 1: bit 0
    blk[20:24] = np.array([0, 0, 1, 0], dtype=np.uint8)        # plane 2: bit 16
    qblk = torch.from_numpy(blk.reshape(1, 24))
    codes = O.sb6_codes(qblk, 1, 32, 2)
    assert codes[0, 0].item() == 3 + 16 and codes[0, 16].item() == 10 + 32
    assert codes[0, 1:16].sum().item() == 0 and codes[0, 17:].sum().item() == 0
    qsqm = torch.tensor([[5, 0xFD]], dtype=torch.uint8)
    ddm = torch.tensor([[0.5, 0.25]], dtype=torch.float16)
    w = O.sb6_dequantize(qblk, qsqm, ddm, 1, 32, 1, 2)
    assert w[0, 0].item() == 46.75 and w[0, 16].item() == 104.25 and w[0, 1].item() == -0.75
    sc, _ = O.sb6_scale_min(qsqm, torch.tensor([[-0.5, 0.25]], dtype=torch.float16), 1, 32, 1,
                            clamp=True)
    assert sc[0, 0].item() == pytest.approx(1e-8)   # max(scale, 1e-8) of the native repack


def test_sb6_repack_equals_affine_dequantize(O):
    """The native repack (codes into the MLX bitstream at 4+xbits bits, fp32
    scale/bias, group 32) dequantizes, through the affine oracle, to exactly
    the sb6 dense weight: MLX's fp32 s*q then +b is the same single rounding."""
    import sb6_k3 as k3
    R, K, gw_sb, xbits = 5, 256, 2, 2
    codes, qs, qm, d, dm = k3.random_sb6(R, K, xbits, gw_sb, seed=11)
    zero = qs == 0          # scale 0: the repack stores max(0, 1e-8) instead
    assert zero.any() and not zero.all()
    qblk, qsqm, ddm = k3.encode(codes, qs, qm, d, dm, xbits)
    wq = O.pack(O.sb6_codes(qblk, R, K, xbits), 4 + xbits)
    sc, mn = O.sb6_scale_min(qsqm, ddm, R, K, gw_sb, clamp=True)
    got = O.dequantize(wq, sc, mn, 32, 4 + xbits)
    want = O.sb6_dequantize(qblk, qsqm, ddm, R, K, gw_sb, xbits)
    same = ~torch.from_numpy(np.repeat(zero, 32, axis=1))
    assert torch.equal(got[same].view(torch.int32), want[same].view(torch.int32))
    clamped = torch.from_numpy(codes).float() * np.float32(1e-8) + want  # want = min there
    assert torch.equal(got[~same], clamped[~same])


# ------------------------------------------------- the CPU-baseline GEMV

def _codes_exact(wq, bits, K):
    """Codes by Python big-integer extraction (independent of the C unpack)."""
    words = wq.view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    out = []
    for r in range(words.shape[0]):
        row = sum(int(words[r, i]) << (32 * i) for i in range(words.shape[1]))
        out.append([(row >> (k * bits)) & ((1 << bits) - 1) for k in range(K)])
    return torch.tensor(out, dtype=torch.float64)


def _qmv_bf16_bound(y, x, we):
    """rqo_qmv_bf16 rounds once to bf16 at the end (2^-9 relative) after fp32
    per-group sums (each within ~gs * 2^-24 of the sum of |terms|); the bound
    is the sum of both, elementwise."""
    ref = x.double() @ we.t()
    mag = x.double().abs() @ we.abs().t()
    err = (y.double() - ref).abs()
    assert bool((err <= 2.0 ** -8 * ref.abs() + 1e-5 * mag).all()), float(
        (err / (2.0 ** -8 * ref.abs() + 1e-5 * mag)).max())
    return ref


@pytest.mark.parametrize("gs", GROUPS)
@pytest.mark.parametrize("bits", BITS)
def test_qmv_bf16_matches_exact_weights_float64(O, bits, gs):
    """rqo_qmv_bf16, the GEMV the CPU baseline times (per-group sums of
    x*code and of x, then scale and bias once per group), against a float64
    product of s*q + b from big-integer-extracted codes, and against
    rqo_qmm's exact-weight mode: the same number up to the final bf16
    rounding."""
    g = torch.Generator().manual_seed(700 + 10 * bits + gs)
    R, K = 24, 512
    w = (torch.randn(R, K, generator=g) * 0.02).to(torch.bfloat16)
    wq, s, b = O.quantize(w, gs, bits)
    we = (_codes_exact(wq, bits, K) * s.double().repeat_interleave(gs, 1)
          + b.double().repeat_interleave(gs, 1))
    for M in (1, 3, 16):
        x = torch.randn(M, K, generator=g).to(torch.bfloat16)
        y = O.qmv_bf16(x, wq, s, b, gs, bits)
        assert y.dtype == torch.bfloat16 and y.shape == (M, R)
        ref = _qmv_bf16_bound(y, x, we)
        ye = O.quantized_matmul(x, wq, s, b, True, gs, bits, out_dtype=torch.float32,
                                weights="exact").double()
        assert torch.allclose(ye, ref, rtol=1e-6, atol=1e-7)
        assert ((y.double() - ye).abs() <= 2.0 ** -8 * ye.abs() + 1e-5).all()


@pytest.mark.parametrize("name,R,K", [("r", 2048, 2048), ("ffn_key", 8192, 2048),
                                      ("ffn_value", 2048, 8192)])
def test_qmv_bf16_config2_shapes(O, name, R, K):
    """The baseline's sample is one RWKV-7 1.5B layer at M = 1: every output
    of each projection within the bound above of the exact-weight product,
    and a dropped bias term or a bias applied to the wrong group would miss it
    (bias * sum(x) over a group is ~10x the per-group dot product here)."""
    g = torch.Generator().manual_seed(2_000_000 + R + K)
    w = (torch.randn(R, K, generator=g) * 0.02).to(torch.bfloat16)
    wq, s, b = O.quantize(w, 64, 4)
    x = torch.randn(1, K, generator=g).to(torch.bfloat16)
    y = O.qmv_bf16(x, wq, s, b, 64, 4)
    ye = O.quantized_matmul(x, wq, s, b, True, 64, 4, out_dtype=torch.float32,
                            weights="exact").double()
    mag = (x.double().abs() @ O.dequantize(wq, s, b, 64, 4, out_dtype=torch.float32).double().abs().t())
    assert ((y.double() - ye).abs() <= 2.0 ** -8 * ye.abs() + 1e-5 * mag).all()
    # the bias contribution is what the per-group factorisation must not lose
    no_bias = O.quantized_matmul(x, wq, s, torch.zeros_like(b), True, 64, 4,
                                 out_dtype=torch.float32, weights="exact").double()
    assert ((no_bias - ye).norm() / ye.norm()).item() > 0.5


# ------------------------------------------------------- exact .5 ties

def _numpy_quantize_ties(w, gs, bits):
    """Group-affine quantize in numpy float32 (IEEE ops, independent of the C
    oracle): codes and the number of exact half-integer quotients rounded."""
    nb = np.float32((1 << bits) - 1)
    a = w.float().numpy().reshape(w.shape[0], -1, gs)
    wmin, wmax = a.min(-1), a.max(-1)
    scale = np.maximum((wmax - wmin) / nb, np.float32(1e-7)).astype(np.float32)
    side = np.abs(wmin) > np.abs(wmax)
    scale = np.where(side, scale, -scale).astype(np.float32)
    edge = np.where(side, wmin, wmax).astype(np.float32)
    e = (edge / scale).astype(np.float32)
    q0 = np.rint(e)
    nz = q0 != 0
    scale = np.where(nz, edge / np.where(nz, q0, np.float32(1)), scale).astype(np.float32)
    bias = np.where(nz, edge, np.float32(0)).astype(np.float32)
    v = ((a - bias[..., None]) / scale[..., None]).astype(np.float32)
    ties = int(((e - np.floor(e)) == 0.5).sum() + ((v - np.floor(v)) == 0.5).sum())
    codes = np.clip(np.rint(v), 0, nb).astype(np.uint8).reshape(w.shape)
    return codes, ties


def test_tie_count_pinned_by_numpy_config1(O):
    """rqo_count_ties against an independent numpy float32 statement of the
    quantizer on benchmark config 1 (RWKV-7 0.1B FFN key [3072, 768], 4-bit
    g64), whose codes must also equal the oracle's bit for bit."""
    g = torch.Generator().manual_seed(1_000_004)
    w = (torch.randn(3072, 768, generator=g) * 0.02).to(torch.bfloat16)
    codes, ties = _numpy_quantize_ties(w, 64, 4)
    wq, _, _ = O.quantize(w, 64, 4)
    assert np.array_equal(O.unpack(wq, 4).numpy(), codes)
    n = O.count_ties(w, 64, 4)
    assert n == ties
    print(f"\nconfig 1 [3072, 768] 4-bit g64: {n} exact .5 quotients of "
          f"{w.numel() + w.numel() // 64} rounded ({100.0 * n / w.numel():.3f} %)")


@pytest.mark.parametrize("bits", BITS)
def test_tie_count_pinned_by_numpy_every_width(O, bits):
    g = torch.Generator().manual_seed(77 + bits)
    w = (torch.randn(256, 1024, generator=g) * 0.02).to(torch.bfloat16)
    codes, ties = _numpy_quantize_ties(w, 64, bits)
    wq, _, _ = O.quantize(w, 64, bits)
    assert np.array_equal(O.unpack(wq, bits).numpy(), codes)
    assert O.count_ties(w, 64, bits) == ties


def test_tie_count_config2_layer_and_head(O):
    """How many codes of a config-2 layer (RWKV-7 1.5B: r/k/v/o, ffn_key,
    ffn_value) and the head are exact .5 ties, i.e. depend on half-to-even
    (MLX's CPU backend, which this oracle and the HIP quantizer follow) versus
    half-away-from-zero rounding.  Reported; a tie count of zero would have
    made the choice moot."""
    total, elems = 0, 0
    for i, (R, K) in enumerate([(2048, 2048)] * 4 + [(8192, 2048), (2048, 8192), (65536, 2048)]):
        g = torch.Generator().manual_seed(2_000_000 + i)
        w = (torch.randn(R, K, generator=g) * 0.02).to(torch.bfloat16)
        total += O.count_ties(w, 64, 4)
        elems += R * K
    assert total > 0
    print(f"\nconfig 2 layer + head, 4-bit g64: {total} exact .5 quotients over {elems} "
          f"weights ({100.0 * total / elems:.3f} %)")

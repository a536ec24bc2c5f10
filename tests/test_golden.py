"""Committed golden vectors (tests/golden/golden.npz, written by
tests/golden/make_golden.py): the oracle must keep reproducing them bit for
bit (CPU), and the HIP library must match them -- quantize, pack and
dequantize bit-exact, quantized_matmul within rel-err 1e-2 (GPU)."""
import hashlib
import os

import numpy as np
import pytest
import torch

from golden import make_golden as G  # tests/golden/make_golden.py

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz")
CASES = [(b, g) for b in G.BITS for g in G.GROUPS]


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLDEN) as z:   # allow_pickle stays False
        return {k: z[k] for k in z.files}


def t16(a, dtype=torch.bfloat16):
    return torch.from_numpy(a.view(np.int16).copy()).view(dtype)


def sha(t):
    return hashlib.sha256(t.cpu().contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()


@pytest.mark.parametrize("bits,gs", CASES)
def test_oracle_reproduces_tiny(O, gold, bits, gs):
    k = f"tiny_b{bits}_g{gs}"
    w = G.tiny_weights(bits, gs)
    x, dy = G.tiny_acts(bits, gs)
    assert np.array_equal(G.bits16(w), gold[f"{k}_w"])
    assert np.array_equal(G.bits16(x), gold[f"{k}_x"])
    wq, s, b = O.quantize(w, gs, bits)
    assert np.array_equal(G.words(wq), gold[f"{k}_wq"])
    assert np.array_equal(G.bits16(s), gold[f"{k}_scales"])
    assert np.array_equal(G.bits16(b), gold[f"{k}_biases"])
    assert np.array_equal(G.bits16(O.dequantize(wq, s, b, gs, bits)), gold[f"{k}_deq"])
    y = O.quantized_matmul(x, wq, s, b, True, gs, bits, out_dtype=torch.float32)
    dx = O.quantized_matmul(dy, wq, s, b, False, gs, bits, out_dtype=torch.float32)
    assert np.array_equal(y.numpy().view(np.uint32), gold[f"{k}_y"].view(np.uint32))
    assert np.array_equal(dx.numpy().view(np.uint32), gold[f"{k}_dx"].view(np.uint32))


def test_oracle_reproduces_config1(O, gold):
    w, x = G.config1_inputs()
    wq, s, b = O.quantize(w, 64, 4)
    deq = O.dequantize(wq, s, b, 64, 4)
    assert [sha(wq), sha(s), sha(b), sha(deq)] == list(gold["config1_sha256"])
    y = O.quantized_matmul(x, wq, s, b, True, 64, 4, out_dtype=torch.float32)
    assert np.array_equal(y.numpy().view(np.uint32), gold["config1_y"].view(np.uint32))


def _rel(y, ref):
    y, ref = y.double().cpu(), ref.double()
    return ((y - ref).norm() / ref.norm()).item(), ((y - ref).abs().max() / ref.abs().max()).item()


@pytest.mark.gpu
@pytest.mark.parametrize("bits,gs", CASES)
def test_hip_matches_tiny(rq, dev, gold, bits, gs):
    k = f"tiny_b{bits}_g{gs}"
    print(f"golden {k}", flush=True)
    w = t16(gold[f"{k}_w"]).to(dev)
    wq, s, b = rq.quantize(w, gs, bits)
    assert np.array_equal(G.words(wq.cpu()), gold[f"{k}_wq"])
    assert np.array_equal(G.bits16(s.cpu()), gold[f"{k}_scales"])
    assert np.array_equal(G.bits16(b.cpu()), gold[f"{k}_biases"])
    assert np.array_equal(G.bits16(rq.dequantize(wq, s, b, gs, bits).cpu()), gold[f"{k}_deq"])
    codes = rq.unpack_codes(wq, bits)
    assert np.array_equal(G.words(rq.pack_codes(codes, bits).cpu()), gold[f"{k}_wq"])
    x, dy = t16(gold[f"{k}_x"]), t16(gold[f"{k}_dy"])
    y = rq.quantized_matmul(x.to(dev), wq, s, b, True, gs, bits).double().cpu()
    dx = rq.quantized_matmul(dy.to(dev), wq, s, b, False, gs, bits).double().cpu()
    y_ref, dx_ref = (torch.from_numpy(gold[f"{k}_{n}"]).double() for n in ("y", "dx"))
    # Row 2 of W is N(0, 1e3).  The oracle rounds s*q and then +b to bf16
    # (MLX's dequantize); the GEMM rounds s*q+b once and the GEMV not at all.
    # Either way a dequantized weight carries an error of up to an ulp of
    # |s*q| + |b|, which near the zero crossings of that row is larger than
    # the weight itself and, through the cancelling dot products, moves y by
    # a few percent.  Every element is therefore bounded by 1e-2 of
    # sum |a| (|s| q + |b|) -- the magnitude the arithmetic works at -- and
    # the usual relative bar is applied to the other rows.
    q = codes.double().cpu()
    sd = t16(gold[f"{k}_scales"]).double().repeat_interleave(gs, 1)
    bd = t16(gold[f"{k}_biases"]).double().repeat_interleave(gs, 1)
    span = sd.abs() * q + bd.abs()
    assert ((y - y_ref).abs() <= 1e-2 * (x.double().abs() @ span.t())).all()
    assert ((dx - dx_ref).abs() <= 1e-2 * (dy.double().abs() @ span)).all()
    keep = [0, 1, 3]
    fro, elem = _rel(y[:, keep], y_ref[:, keep])
    assert fro <= 1e-2 and elem <= 1e-2, ("y", fro, elem)
    dy0 = dy.clone()
    dy0[:, 2] = 0   # drop row 2 of W from the contraction
    dx0 = rq.quantized_matmul(dy0.to(dev), wq, s, b, False, gs, bits).double().cpu()
    fro, elem = _rel(dx0, dy0.double() @ t16(gold[f"{k}_deq"]).double())
    assert fro <= 1e-2 and elem <= 1e-2, ("dx without row 2", fro, elem)


@pytest.mark.gpu
def test_hip_matches_config1(rq, dev, gold):
    print("golden config1", flush=True)
    w, x = G.config1_inputs()
    wq, s, b = rq.quantize(w.to(dev), 64, 4)
    deq = rq.dequantize(wq, s, b, 64, 4)
    assert [sha(wq), sha(s), sha(b), sha(deq)] == list(gold["config1_sha256"])
    for m in (1, 16):
        y = rq.quantized_matmul(x[:m].to(dev), wq, s, b, True, 64, 4)
        fro, elem = _rel(y, torch.from_numpy(gold["config1_y"][:m]))
        assert fro <= 1e-2 and elem <= 1e-2, (m, fro, elem)

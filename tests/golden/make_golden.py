"""Write tests/golden/golden.npz: fixed input/output vectors of the CPU oracle.

The reference's own tests commit no vectors for this path (its checks need
MLX and checkpoint files that are not part of it), so these fixtures freeze
the oracle's outputs -- after the oracle itself has been checked against the
rule text, the probe KAT and the closed forms in tests/test_oracle.py -- so
that any later change to the oracle or to the GPU kernels is caught bit for
bit.  Inputs are regenerated from the seeds below and also stored.

Cases:
  tiny_b{bits}_g{gs}: W [4, 256] (random, constant/zero, wide-range and tie
      rows), x [3, 256], dY [3, 4]; outputs w_q, scales, biases, dequantized
      W, y = x . W^T and dX = dY . W (fp32, oracle's float64 accumulation).
  config1: W [3072, 768] 4-bit g64 (the 0.1B FFN key) and x [16, 768]:
      SHA-256 of w_q / scales / biases / dequantized bytes, and y in fp32.

Run: python tests/golden/make_golden.py  (needs the oracle: make -C oracle)
"""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

OUT = os.path.join(HERE, "golden.npz")
BITS = (2, 3, 4, 5, 6, 8)
GROUPS = (32, 64, 128)


def tiny_weights(bits: int, gs: int) -> torch.Tensor:
    K = 256
    g = torch.Generator().manual_seed(7_000 + 10 * bits + gs)
    rows = [
        torch.randn(K, generator=g) * 0.02,
        torch.cat([torch.full((K // 2,), 0.37), torch.zeros(K // 2)]),
        torch.randn(K, generator=g) * 1e3,
        torch.linspace(-1.0, 1.0, K),
    ]
    return torch.stack(rows).to(torch.bfloat16)


def tiny_acts(bits: int, gs: int):
    g = torch.Generator().manual_seed(8_000 + 10 * bits + gs)
    x = torch.randn(3, 256, generator=g).to(torch.bfloat16)
    dy = torch.randn(3, 4, generator=g).to(torch.bfloat16)
    return x, dy


def config1_inputs():
    w = (torch.randn(3072, 768, generator=torch.Generator().manual_seed(1_000_004)) * 0.02
         ).to(torch.bfloat16)
    x = torch.randn(16, 768, generator=torch.Generator().manual_seed(1_000_504)).to(torch.bfloat16)
    return w, x


def bits16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def words(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int32).numpy().view(np.uint32)


def sha(t: torch.Tensor) -> str:
    return hashlib.sha256(t.contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()


def main() -> None:
    from oracle import oracle as O
    if not os.path.exists(O._LIB_PATH):
        O.build()
    arrays = {}
    for bits in BITS:
        for gs in GROUPS:
            k = f"tiny_b{bits}_g{gs}"
            w = tiny_weights(bits, gs)
            x, dy = tiny_acts(bits, gs)
            wq, s, b = O.quantize(w, gs, bits)
            deq = O.dequantize(wq, s, b, gs, bits)
            y = O.quantized_matmul(x, wq, s, b, True, gs, bits, out_dtype=torch.float32)
            dx = O.quantized_matmul(dy, wq, s, b, False, gs, bits, out_dtype=torch.float32)
            arrays.update({f"{k}_w": bits16(w), f"{k}_x": bits16(x), f"{k}_dy": bits16(dy),
                           f"{k}_wq": words(wq), f"{k}_scales": bits16(s),
                           f"{k}_biases": bits16(b), f"{k}_deq": bits16(deq),
                           f"{k}_y": y.numpy(), f"{k}_dx": dx.numpy()})
    w, x = config1_inputs()
    wq, s, b = O.quantize(w, 64, 4)
    deq = O.dequantize(wq, s, b, 64, 4)
    y = O.quantized_matmul(x, wq, s, b, True, 64, 4, out_dtype=torch.float32)
    arrays["config1_sha256"] = np.array([sha(wq), sha(s), sha(b), sha(deq)])
    arrays["config1_y"] = y.numpy()
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes, {len(arrays)} arrays)")


if __name__ == "__main__":
    main()

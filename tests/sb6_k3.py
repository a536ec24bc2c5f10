"""K3-interleaved sb6 test data, encoded straight from the layout the
reference states (rwkv_metal/lora/rwkvq_kernel.py:18-25 and the decode in
rwkv_metal/lora/rwkvq_linear.py:140-175):

  qblk[row, blk] : 16 bytes, byte j = (code j & 15) | (code j+16 & 15) << 4;
                   xbits >= 1: a little-endian uint32, bit c = bit 4 of code c;
                   xbits == 2: another, bit c = bit 5 of code c
  qsqm[row, blk] : (qs uint8, qm int8 as its byte)
  ddm[row, sblk] : (d, dm) float16, sblk = blk // gw_sb
  scale = f16(qs * d), min = f16(qm * dm), w = code * scale + min (fp32)

numpy only; used by the oracle pins (CPU) and the GPU parity tests.
"""
import numpy as np
import torch


def encode(codes, qs, qm, d, dm, xbits):
    """codes int[R, K] (< 2^(4+xbits)), qs uint8[R, NB], qm int8[R, NB],
    d/dm float16[R, NSB] -> (qblk uint8[R, NB*(16+4*xbits)], qsqm uint8[R, 2*NB],
    ddm float16[R, 2*NSB]) as torch tensors."""
    codes = np.asarray(codes, dtype=np.int64)
    R, K = codes.shape
    NB = K // 32
    blk = codes.reshape(R, NB, 32)
    lo = (blk[:, :, :16] & 15) | ((blk[:, :, 16:] & 15) << 4)
    parts = [lo.astype(np.uint8)]
    for x in range(xbits):
        plane = np.zeros((R, NB), dtype=np.uint64)
        for c in range(32):
            plane |= (((blk[:, :, c] >> (4 + x)) & 1).astype(np.uint64) << np.uint64(c))
        parts.append(plane.astype("<u4").view(np.uint8).reshape(R, NB, 4))
    qblk = np.concatenate(parts, axis=2).reshape(R, NB * (16 + 4 * xbits))
    qsqm = np.stack([np.asarray(qs, np.uint8), np.asarray(qm, np.int8).view(np.uint8)],
                    axis=2).reshape(R, 2 * NB)
    ddm = np.stack([np.asarray(d, np.float16), np.asarray(dm, np.float16)], axis=2).reshape(R, -1)
    return (torch.from_numpy(np.ascontiguousarray(qblk)), torch.from_numpy(np.ascontiguousarray(qsqm)),
            torch.from_numpy(np.ascontiguousarray(ddm)))


def scale_min(qs, qm, d, dm, gw_sb, clamp=False):
    """fp32 [R, NB]: f16(qs*d), f16(qm*dm) (numpy float32 products, RNE to f16)."""
    d_c = np.repeat(np.asarray(d, np.float16).astype(np.float32), gw_sb, axis=1)
    dm_c = np.repeat(np.asarray(dm, np.float16).astype(np.float32), gw_sb, axis=1)
    sc = (np.asarray(qs, np.uint8).astype(np.float32) * d_c).astype(np.float16).astype(np.float32)
    mn = (np.asarray(qm, np.int8).astype(np.float32) * dm_c).astype(np.float16).astype(np.float32)
    if clamp:
        sc = np.maximum(sc, np.float32(1e-8))
    return sc, mn


def dense(codes, qs, qm, d, dm, gw_sb):
    """fp32 [R, K]: code * scale + min with separate fp32 multiply and add."""
    sc, mn = scale_min(qs, qm, d, dm, gw_sb)
    c = np.asarray(codes, np.float32)
    R, K = c.shape
    return (c * np.repeat(sc, 32, axis=1)).astype(np.float32) + np.repeat(mn, 32, axis=1)


def random_sb6(R, K, xbits, gw_sb, seed, tiny=False):
    """Random codes and block parameters shaped like a calibrated sb6 tensor:
    qs 6-bit, qm in [-31, 32] (int8 after the export's -31 shift), d and dm
    small positive float16 (some subnormal when tiny=True)."""
    rng = np.random.default_rng(seed)
    NB, NSB = K // 32, K // 32 // gw_sb
    codes = rng.integers(0, 1 << (4 + xbits), size=(R, K))
    qs = rng.integers(0, 64, size=(R, NB)).astype(np.uint8)
    qm = (rng.integers(0, 64, size=(R, NB)) - 31).astype(np.int8)
    d = (rng.random((R, NSB)) * 2e-3 + 1e-4).astype(np.float16)
    dm = (-(rng.random((R, NSB)) * 2e-3 + 1e-4)).astype(np.float16)
    if tiny:
        d[:, ::3] = np.float16(3e-7)    # subnormal float16 super-block scales
        dm[:, ::2] = np.float16(-6e-8)
    return codes, qs, qm, d, dm

"""fp32 activations on the fast GEMMs (the reference's default: the residual
stream is fp32, rwkv_metal/model/rwkv7_x070.py:51,189-194, and
RwkvqNativeLinear casts x to fp32, rwkv_metal/lora/rwkvq_native.py:120).

The 64-wide-stage GEMMs, the one-launch QLoRA products and the adapter
gradients round fp32 x / dY to bf16 as they stage them, so each fp32 result
must equal, bit for bit, the bf16 path run on bf16(x) with the same output
dtype; and it must sit within the 1e-2 bar of the fp32 product (the oracle,
or an fp32 dense reference at sizes the oracle is too slow for)."""
import pytest
import torch

from test_gpu_parity import acts, bits_equal, rel_check, say, weights

pytestmark = pytest.mark.gpu


def _abi_qmm(x, wq, s, b, transpose, gs, bits, y_dt=torch.float32):
    """rq_qmm through the C ABI with an explicit output dtype."""
    from rwkvq._lib import DTYPE_CODE, lib
    from rwkvq.ops import _stream_on
    R, K = wq.shape[0], wq.shape[1] * 32 // bits
    m = x.shape[0]
    y = torch.full((m, R if transpose else K), float("nan"), dtype=y_dt, device=x.device)
    rc = lib().rq_qmm(x.data_ptr(), DTYPE_CODE[x.dtype], wq.data_ptr(), s.data_ptr(),
                      b.data_ptr(), DTYPE_CODE[s.dtype], m, R, K, gs, bits,
                      1 if transpose else 0, y.data_ptr(), DTYPE_CODE[y_dt], _stream_on(x.device))
    assert rc == 0, lib().rq_last_error().decode()
    return y


# (transpose, M, R, K, bits, gs, scales dtype): 256-, 128- and 64-row tiles of
# the forward GEMM, 128- and 160-column tiles of the transposed one, partial
# tiles, 3/4/8-bit codes, every group size, f16 scales
CASES = [
    (True, 4096, 2560, 2560, 4, 64, torch.bfloat16),
    (True, 2048, 2560, 2560, 4, 64, torch.bfloat16),
    (True, 512, 2560, 2560, 4, 64, torch.bfloat16),
    (True, 1100, 10240, 1024, 3, 64, torch.bfloat16),
    (True, 700, 2048, 512, 8, 32, torch.float16),
    (True, 300, 520, 1024, 4, 128, torch.bfloat16),
    (False, 4096, 2048, 2048, 4, 64, torch.bfloat16),
    (False, 4096, 2560, 2560, 4, 64, torch.bfloat16),
    (False, 700, 320, 960, 8, 32, torch.float16),
    (False, 300, 256, 512, 3, 64, torch.bfloat16),
]


@pytest.mark.parametrize("transpose,M,R,K,bits,gs,sdt", CASES)
def test_fp32_x_equals_bf16_rounded_x(rq, dev, transpose, M, R, K, bits, gs, sdt):
    """fp32 x (transpose=1) / fp32 dY (transpose=0) at M >= 256: the same
    bits as bf16(x) through the bf16 kernels with an fp32 output, and within
    the bar of the fp32 dense product."""
    say(f"fp32 x t={transpose} M={M} R={R} K={K} b={bits} gs={gs} s={sdt}")
    wq, s, b = rq.quantize(weights(R, K, 90_000 + R + K + bits, sdt).to(dev), gs, bits)
    n_in = K if transpose else R
    x = acts(M, n_in, 91_000 + M + bits, torch.float32).to(dev)
    y32 = _abi_qmm(x, wq, s, b, transpose, gs, bits)
    yb = _abi_qmm(x.to(torch.bfloat16), wq, s, b, transpose, gs, bits)
    assert bits_equal(y32, yb), "fp32-x result differs from the bf16(x) one"
    # the torch op: MLX promotion (fp32 x with 16-bit scales gives fp32)
    y = rq.quantized_matmul(x, wq, s, b, transpose, gs, bits)
    assert y.dtype == torch.float32 and bits_equal(y, y32)
    q = rq.unpack_codes(wq, bits).float()
    wd = q * s.float().repeat_interleave(gs, 1) + b.float().repeat_interleave(gs, 1)
    rel_check(y32, x @ (wd.t() if transpose else wd), what="fp32 x vs fp32 dense")


def test_fp32_x_against_oracle(O, rq, dev):
    """One fp32-x problem on the 256-row tiles against the CPU oracle's fp32
    product (weights s*q + b unrounded)."""
    M, R, K = 800, 10240, 512
    w = weights(R, K, 92)
    wq, s, b = O.quantize(w, 64, 4)
    x = acts(M, K, 93, torch.float32)
    say("fp32 x vs oracle")
    y = rq.quantized_matmul(x.to(dev), wq.to(dev), s.to(dev), b.to(dev), True, 64, 4)
    rel_check(y, O.quantized_matmul(x, wq, s, b, True, 64, 4, out_dtype=torch.float32,
                                    weights="exact"), what="fp32 x oracle")


@pytest.mark.parametrize("transpose,M,R,K", [(True, 4096, 2048, 2048), (True, 4096, 8192, 2048),
                                             (False, 4096, 2048, 8192), (False, 700, 320, 1024)])
def test_qlora_fp32_x_one_launch(rq, dev, transpose, M, R, K):
    """rq_qlora with fp32 x / dY: y (fp32) and z bit-identical to the bf16(x)
    launch with an fp32 output."""
    from rwkvq import _lib, ops
    from rwkvq.ops import _stream_on
    say(f"qlora fp32 x t={transpose} M={M} R={R} K={K}")
    wq, s, b = rq.quantize(weights(R, K, 94_000 + R).to(dev), 64, 4)
    n_in, n_out = (K, R) if transpose else (R, K)
    g = torch.Generator().manual_seed(M + R)
    x = acts(M, n_in, 95_000 + M, torch.float32).to(dev)
    a = (torch.randn(16, n_in, generator=g) / n_in ** 0.5).to(torch.bfloat16).to(dev)
    L = (torch.randn(n_out, 16, generator=g) * 0.05).to(torch.bfloat16).to(dev)
    yz = ops.qlora_fused(x, wq, s, b, a, L, 0.75, transpose, 64, 4)
    assert yz is not None, "fp32 x must run the one-launch kernels"
    y, z = yz
    assert y.dtype == torch.float32 and z.dtype == torch.bfloat16
    xb = x.to(torch.bfloat16)
    yb = torch.empty_like(y)
    zb = torch.empty_like(z)
    rc = _lib.lib().rq_qlora(xb.data_ptr(), _lib.RQ_BF16, wq.data_ptr(), s.data_ptr(), b.data_ptr(),
                             _lib.RQ_BF16, M, R, K, 64, 4, 1 if transpose else 0, a.data_ptr(),
                             L.data_ptr(), 16, 0.75, zb.data_ptr(), yb.data_ptr(), _lib.RQ_F32,
                             _stream_on(dev))
    assert rc == 0, _lib.lib().rq_last_error().decode()
    assert bits_equal(z, zb) and bits_equal(y, yb)


@pytest.mark.parametrize("M,K,N,rank", [(4096, 2048, 8192, 16), (1000, 520, 136, 32),
                                        (4097, 64, 2056, 64)])
def test_lora_grads_f32_equals_bf16_rounded(rq, dev, M, K, N, rank):
    """rq_lora_grads_f32 (fp32 x and dY) gives the bits of rq_lora_grads on
    bf16(x) and bf16(dY), and the fp32 products within the bar."""
    from rwkvq import ops
    say(f"lora_grads_f32 M={M} K={K} N={N} rank={rank}")
    g = torch.Generator().manual_seed(M + K + N)
    x = torch.randn(M, K, generator=g).to(dev)
    u = torch.randn(M, rank, generator=g).to(torch.bfloat16).to(dev)
    dy = torch.randn(M, N, generator=g).to(dev)
    z = torch.randn(M, rank, generator=g).to(torch.bfloat16).to(dev)
    da, db = ops.lora_grads(x, u, dy, z, 0.5)
    dab, dbb = ops.lora_grads(x.to(torch.bfloat16), u, dy.to(torch.bfloat16), z, 0.5)
    assert bits_equal(da, dab) and bits_equal(db, dbb)
    rel_check(da, 0.5 * (u.float().t() @ x), what="dA")
    rel_check(db, 0.5 * (dy.t() @ z.float()), what="dB")


def test_config4_qlora_layer_step_fp32_x(rq, dev):
    """Benchmark config 4 with the reference's fp32 activations: one RWKV-7
    1.5B layer (D = 2048) on a frozen 4-bit g64 base, 8 x 512 tokens, r =
    alpha = 16; y, dX, dA and dB of every projection against an fp32 dense
    reference on the dequantized base, with the fused kernels running (y is
    fp32, dX is fp32)."""
    from rwkvq import ops
    D, F, r, alpha = 2048, 8192, 16, 16.0
    for i, (name, R, K) in enumerate([("r", D, D), ("ffn_key", F, D), ("ffn_value", D, F)]):
        say(f"config4 fp32-x layer step {name} [{R},{K}]")
        base = rq.QuantizedLinear(K, R, bias=False, group_size=64, bits=4, device=dev)
        wq, s, b = rq.quantize(weights(R, K, 4_100_000 + i).to(dev), 64, 4)
        base.weight, base.scales, base.biases = wq, s, b
        lay = rq.LoRALinear(rank=r, alpha=alpha, base_module=base)
        g = torch.Generator().manual_seed(4_100_600 + i)
        with torch.no_grad():
            lay.lora_a.copy_((torch.randn(r, K, generator=g) / K ** 0.5).to(torch.bfloat16))
            lay.lora_b.copy_((torch.randn(R, r, generator=g) * 0.01).to(torch.bfloat16))
        x = acts(8 * 512, K, 4_100_000 + i, torch.float32).to(dev).reshape(8, 512, K)
        x.requires_grad_(True)
        dy = acts(8 * 512, R, 4_100_800 + i, torch.float32).to(dev).reshape(8, 512, R)
        assert lay._fusable(x)
        assert ops.qlora_fused(x.detach().reshape(-1, K), wq, s, b, lay.lora_a.detach(),
                               lay.lora_b.detach(), 1.0, True, 64, 4) is not None
        y = lay(x)
        assert y.dtype == torch.float32
        dx, da, db = torch.autograd.grad(y, (x, lay.lora_a, lay.lora_b), dy)
        assert dx.dtype == torch.float32 and da.dtype == db.dtype == torch.bfloat16
        q = rq.unpack_codes(wq, 4).float()
        wd = q * s.float().repeat_interleave(64, 1) + b.float().repeat_interleave(64, 1)
        xr = x.detach().reshape(-1, K).clone().requires_grad_(True)
        A = lay.lora_a.detach().float().requires_grad_(True)
        B = lay.lora_b.detach().float().requires_grad_(True)
        yr = xr @ wd.t() + (alpha / r) * ((xr @ A.t()) @ B.t())
        yr.backward(dy.reshape(-1, R))
        rel_check(y.reshape(-1, R), yr, what=f"{name} y")
        rel_check(dx.reshape(-1, K), xr.grad, what=f"{name} dX")
        rel_check(da, A.grad, what=f"{name} dA")
        rel_check(db, B.grad, what=f"{name} dB")

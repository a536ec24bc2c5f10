"""GPU parity of the QLoRA layer's kernels (rwkv_metal/lora/lora.py:58-63 under
nn.value_and_grad, rwkv_metal/lora/finetune.py:141): the adapter-gradient
launch rq_lora_grads against fp32 products of the same bf16 operands, and the
whole layer step at benchmark config 4's full size against an fp32 dense
reference on the dequantized base."""
import pytest
import torch

from test_gpu_parity import acts, bits_equal, rel_check, say, weights

pytestmark = pytest.mark.gpu


def _grads_ref(x, u, dy, z, scale):
    da = scale * (u.float().t() @ x.float()) if x is not None else None
    db = scale * (dy.float().t() @ z.float()) if dy is not None else None
    return da, db


# (M, K, N, rank): one chunk per tile (few rows), several chunks with a
# partial last one, ragged column tiles (K, N multiples of 8, not 64), the
# config-4 shapes
GRAD_CASES = [
    (40, 256, 128, 16),
    (1000, 520, 136, 32),
    (4096, 2048, 2048, 16),
    (4096, 2048, 8192, 16),
    (4096, 8192, 2048, 64),
    (3000, 1024, 4096, 48),
    (4097, 64, 2056, 16),
]


@pytest.mark.parametrize("M,K,N,rank", GRAD_CASES)
def test_lora_grads_matches_fp32(rq, dev, M, K, N, rank):
    from rwkvq import ops
    say(f"lora_grads M={M} K={K} N={N} rank={rank}")
    g = torch.Generator().manual_seed(M + K + N + rank)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
    u = torch.randn(M, rank, generator=g).to(torch.bfloat16).to(dev)
    dy = torch.randn(M, N, generator=g).to(torch.bfloat16).to(dev)
    z = torch.randn(M, rank, generator=g).to(torch.bfloat16).to(dev)
    da, db = ops.lora_grads(x, u, dy, z, 0.5)
    assert da.shape == (rank, K) and db.shape == (N, rank) and da.dtype == torch.bfloat16
    rda, rdb = _grads_ref(x, u, dy, z, 0.5)
    rel_check(da, rda, what="dA")
    rel_check(db, rdb, what="dB")
    # deterministic: the partial tiles are summed in chunk order whatever order
    # the chunks finish in, and the counters are back at zero for the next call
    da2, db2 = ops.lora_grads(x, u, dy, z, 0.5)
    assert torch.equal(da2.view(torch.int16), da.view(torch.int16))
    assert torch.equal(db2.view(torch.int16), db.view(torch.int16))
    # one gradient alone (the other pair of operands is not read)
    da3, db3 = ops.lora_grads(x, u, None, None, 0.5)
    assert db3 is None
    rel_check(da3, rda, what="dA alone")
    da4, db4 = ops.lora_grads(None, None, dy, z, 0.5)
    assert da4 is None
    rel_check(db4, rdb, what="dB alone")


def test_lora_grads_empty_contraction_is_zero(rq, dev):
    from rwkvq import ops
    x = torch.empty(0, 256, dtype=torch.bfloat16, device=dev)
    u = torch.empty(0, 16, dtype=torch.bfloat16, device=dev)
    dy = torch.empty(0, 128, dtype=torch.bfloat16, device=dev)
    z = torch.empty(0, 16, dtype=torch.bfloat16, device=dev)
    da, db = ops.lora_grads(x, u, dy, z, 1.0)
    assert da.shape == (16, 256) and db.shape == (128, 16)
    assert not da.float().abs().any() and not db.float().abs().any()


# ------------------------------------------------ one-launch QLoRA products

def _wdense(rq, wq, s, b, gs, bits):
    """fp32 s*q + b from the (bit-exact) unpacked codes: [R, K]."""
    q = rq.unpack_codes(wq, bits).float()
    return q * s.float().repeat_interleave(gs, 1) + b.float().repeat_interleave(gs, 1)


def _dense(rq, x, wq, s, b, gs, bits, transpose):
    wd = _wdense(rq, wq, s, b, gs, bits)
    return x.float() @ (wd.t() if transpose else wd)


# (transpose, M, R, K, bits, gs, scales dtype): 256- and 128-row tiles,
# partial row and column tiles, 4 and 8 bits, every group size, f16 scales
QLORA_CASES = [
    (True, 4096, 2048, 2048, 4, 64, torch.bfloat16),
    (True, 4096, 8192, 2048, 4, 64, torch.bfloat16),
    (True, 4096, 2048, 8192, 4, 64, torch.bfloat16),
    (True, 1000, 520, 1024, 4, 128, torch.bfloat16),
    (True, 300, 2048, 512, 8, 32, torch.float16),
    (False, 4096, 2048, 2048, 4, 64, torch.bfloat16),
    (False, 4096, 8192, 2048, 4, 64, torch.bfloat16),
    (False, 4096, 2048, 8192, 4, 64, torch.bfloat16),
    (False, 700, 320, 1024, 8, 128, torch.float16),
    (False, 300, 256, 512, 4, 32, torch.bfloat16),
]


@pytest.mark.parametrize("transpose,M,R,K,bits,gs,sdt", QLORA_CASES)
def test_qlora_one_launch(rq, dev, transpose, M, R, K, bits, gs, sdt):
    """rq_qlora: z = x a^T computed inside the GEMM (rounded once to bf16,
    stored for the backward) and y = qmm(x) + scale * z lora^T, against fp32
    products of the same bf16 operands."""
    from rwkvq import ops
    say(f"qlora one launch t={transpose} M={M} R={R} K={K} b={bits} gs={gs} s={sdt}")
    wq, s, b = rq.quantize(weights(R, K, 70_000 + R + K, sdt).to(dev), gs, bits)
    n_in, n_out = (K, R) if transpose else (R, K)
    g = torch.Generator().manual_seed(M + R + K)
    x = acts(M, n_in, M + K).to(dev)
    a = (torch.randn(16, n_in, generator=g) / n_in ** 0.5).to(torch.bfloat16).to(dev)
    L = (torch.randn(n_out, 16, generator=g) * 0.05).to(torch.bfloat16).to(dev)
    yz = ops.qlora_fused(x, wq, s, b, a, L, 0.75, transpose, gs, bits)
    assert yz is not None, "this problem must run the one-launch kernels"
    y, z = yz
    zref = x.float() @ a.float().t()
    rel_check(z, zref, what="z")
    # the term uses z rounded to bf16, as the two-launch path does
    ref = _dense(rq, x, wq, s, b, gs, bits, transpose) + 0.75 * (z.float() @ L.float().t())
    rel_check(y, ref, what="y")
    # and the two-launch path gives the same product within the bar
    y2 = ops.quantized_matmul_lora(x, wq, s, b, ops.lora_down(x, a), L, 0.75, transpose, gs, bits)
    rel_check(y, y2.float(), what="y vs lora_down + rq_qmm_lora")


@pytest.mark.parametrize("M,R,K,bits,gs,sdt", [c[1:] for c in QLORA_CASES if not c[0]])
@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float32])
def test_qlora_dx_from_stored_adapters(rq, dev, M, R, K, bits, gs, sdt, xdt):
    """rq_qlora_dx reads lora_a [16, K] and lora_b [R, 16] as the layer
    stores them (strided fragment loads) and must give rq_qlora(transpose=0)'s
    bits on their transposed copies: dX and u = dY lora_b."""
    from rwkvq import ops
    say(f"qlora dx stored adapters M={M} R={R} K={K} b={bits} gs={gs} s={sdt} x={xdt}")
    wq, s, b = rq.quantize(weights(R, K, 71_000 + R + K, sdt).to(dev), gs, bits)
    g = torch.Generator().manual_seed(M + R + K + 1)
    dy = acts(M, R, M + R).to(xdt).to(dev)
    lora_a = (torch.randn(16, K, generator=g) / K ** 0.5).to(torch.bfloat16).to(dev)
    lora_b = (torch.randn(R, 16, generator=g) * 0.05).to(torch.bfloat16).to(dev)
    got = ops.qlora_dx_fused(dy, wq, s, b, lora_a, lora_b, 0.75, gs, bits)
    want = ops.qlora_fused(dy, wq, s, b, lora_b.t().contiguous(), lora_a.t().contiguous(), 0.75,
                           False, gs, bits)
    assert got is not None and want is not None, "this problem must run the one-launch kernels"
    assert bits_equal(got[1], want[1]), "u"
    assert bits_equal(got[0], want[0]), "dX"
    # adapters that are views with gaps are made contiguous, not misread
    wide = torch.zeros(R, 32, dtype=torch.bfloat16, device=dev)
    wide[:, :16] = lora_b
    again = ops.qlora_dx_fused(dy, wq, s, b, lora_a, wide[:, :16], 0.75, gs, bits)
    assert bits_equal(again[0], want[0])


@pytest.mark.parametrize("transpose,M,R,K,bits", [(True, 4096, 8192, 2048, 4),
                                                  (False, 4096, 2048, 8192, 4),
                                                  (True, 512, 4096, 1024, 8),
                                                  (False, 300, 1024, 4096, 8)])
@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float32])
def test_qlora_wide_outputs_take_two_launches(rq, dev, transpose, M, R, K, bits, xdt):
    """Outputs at least 4096 wide and twice the contraction run the
    down-projection as its own pass (x read once) and the term in the GEMM's
    output stage: the forward and both dX entry points give exactly the bits
    of lora_down + quantized_matmul_lora on bf16(x) -- for rq_qlora_dx with B
    read as stored [R, 16] by the pass and A as stored [16, K] by the output
    stage."""
    from rwkvq import ops
    say(f"qlora two launches t={transpose} M={M} R={R} K={K} b={bits} x={xdt}")
    wq, s, b = rq.quantize(weights(R, K, 72_000 + R + K).to(dev), 64, bits)
    n_in, n_out = (K, R) if transpose else (R, K)
    g = torch.Generator().manual_seed(M + R + K + 2)
    x = acts(M, n_in, M + n_in + 2).to(xdt).to(dev)
    xb = x.to(torch.bfloat16)
    lora_a = (torch.randn(16, K, generator=g) / K ** 0.5).to(torch.bfloat16).to(dev)
    lora_b = (torch.randn(R, 16, generator=g) * 0.05).to(torch.bfloat16).to(dev)
    if transpose:
        y, z = ops.qlora_fused(x, wq, s, b, lora_a, lora_b, 0.75, True, 64, bits,
                               out_dtype=torch.float32)
        zr = ops.lora_down(xb, lora_a)
        yr = ops.quantized_matmul_lora(xb, wq, s, b, zr, lora_b, 0.75, True, 64, bits)
    else:
        y, z = ops.qlora_dx_fused(x, wq, s, b, lora_a, lora_b, 0.75, 64, bits,
                                  out_dtype=torch.float32)
        y2, z2 = ops.qlora_fused(x, wq, s, b, lora_b.t().contiguous(), lora_a.t().contiguous(),
                                 0.75, False, 64, bits, out_dtype=torch.float32)
        assert bits_equal(z, z2) and bits_equal(y, y2), "rq_qlora_dx against rq_qlora(transpose=0)"
        zr = ops.lora_down(xb, lora_b.t().contiguous())
        yr = ops.quantized_matmul_lora(xb, wq, s, b, zr, lora_a.t().contiguous(), 0.75, False, 64,
                                       bits)
    assert bits_equal(z, zr), "the down-projection pass"
    assert yr.dtype == torch.bfloat16
    # the GEMM rounds once into y's dtype: compare against the fp32 output of
    # the same two launches
    yr32 = torch.empty_like(y)
    from rwkvq import _lib
    from rwkvq.ops import _stream_on
    lo = lora_b if transpose else lora_a.t().contiguous()
    rc = _lib.lib().rq_qmm_lora(xb.data_ptr(), _lib.RQ_BF16, wq.data_ptr(), s.data_ptr(),
                                b.data_ptr(), _lib.RQ_BF16, M, R, K, 64, bits, 1 if transpose else 0,
                                zr.data_ptr(), lo.data_ptr(), 16, 0.75, yr32.data_ptr(),
                                _lib.RQ_F32, _stream_on(dev))
    assert rc == 0, _lib.lib().rq_last_error().decode()
    assert bits_equal(y, yr32), "the GEMM with the term in its output stage"
    rel_check(yr32, yr.float(), what="fp32 vs bf16 output")


def test_qlora_one_launch_declines_other_ranks_and_bits(rq, dev):
    from rwkvq import ops
    wq, s, b = rq.quantize(weights(256, 512, 3).to(dev), 64, 3)
    x = acts(512, 512, 3).to(dev)
    a = torch.zeros(16, 512, dtype=torch.bfloat16, device=dev)
    L = torch.zeros(256, 16, dtype=torch.bfloat16, device=dev)
    assert ops.qlora_fused(x, wq, s, b, a, L, 1.0, True, 64, 3) is None        # 3-bit codes
    wq, s, b = rq.quantize(weights(256, 512, 4).to(dev), 64, 4)
    a32 = torch.zeros(32, 512, dtype=torch.bfloat16, device=dev)
    L32 = torch.zeros(256, 32, dtype=torch.bfloat16, device=dev)
    assert ops.qlora_fused(x, wq, s, b, a32, L32, 1.0, True, 64, 4) is None    # rank 32
    assert ops.qlora_fused(x[:100], wq, s, b, a, L, 1.0, True, 64, 4) is None  # m < 256


def test_config4_qlora_layer_step_full_size(rq, dev):
    """benchmark config 4 at full size: one RWKV-7 1.5B layer (D = 2048) on a
    frozen 4-bit g64 base, 8 x 512 tokens, r = alpha = 16, A ~ N(0, 1/D),
    B ~ N(0, 0.01) (std); for each of r, k, v, o, ffn_key and ffn_value the
    forward y = qmm(x, Wq) + (alpha / r) (x A^T) B^T and the gradients dX, dA,
    dB against an fp32 dense reference on the dequantized base.  Every
    projection runs the one-launch forward and dX kernels and one
    adapter-gradient launch."""
    D, F, r, alpha = 2048, 8192, 16, 16.0
    for i, (name, R, K) in enumerate([("r", D, D), ("k", D, D), ("v", D, D), ("o", D, D),
                                      ("ffn_key", F, D), ("ffn_value", D, F)]):
        say(f"config4 layer step {name} [{R},{K}]")
        base = rq.QuantizedLinear(K, R, bias=False, group_size=64, bits=4, device=dev)
        wq, s, b = rq.quantize(weights(R, K, 4_000_000 + 1000 + i).to(dev), 64, 4)
        base.weight, base.scales, base.biases = wq, s, b
        lay = rq.LoRALinear(rank=r, alpha=alpha, base_module=base)
        g = torch.Generator().manual_seed(4_000_600 + i)
        with torch.no_grad():
            lay.lora_a.copy_((torch.randn(r, K, generator=g) / K ** 0.5).to(torch.bfloat16))
            lay.lora_b.copy_((torch.randn(R, r, generator=g) * 0.01).to(torch.bfloat16))
        x = acts(8 * 512, K, 4_000_000 + i).to(dev).reshape(8, 512, K).requires_grad_(True)
        dy = acts(8 * 512, R, 4_000_800 + i).to(dev).reshape(8, 512, R)
        from rwkvq import ops
        assert ops.qlora_fused(x.detach().reshape(-1, K), wq, s, b, lay.lora_a.detach(),
                               lay.lora_b.detach(), 1.0, True, 64, 4) is not None
        y = lay(x)
        dx, da, db = torch.autograd.grad(y, (x, lay.lora_a, lay.lora_b), dy)
        wd = _wdense(rq, wq, s, b, 64, 4)
        xr = x.detach().float().reshape(-1, K).requires_grad_(True)
        A = lay.lora_a.detach().float().requires_grad_(True)
        B = lay.lora_b.detach().float().requires_grad_(True)
        yr = xr @ wd.t() + (alpha / r) * ((xr @ A.t()) @ B.t())
        yr.backward(dy.float().reshape(-1, R))
        rel_check(y.reshape(-1, R), yr, what=f"{name} y")
        rel_check(dx.reshape(-1, K), xr.grad, what=f"{name} dX")
        rel_check(da, A.grad, what=f"{name} dA")
        rel_check(db, B.grad, what=f"{name} dB")

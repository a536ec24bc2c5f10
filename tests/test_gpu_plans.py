"""GPU parity of the exact launches bench.py times, and of the fused QLoRA
output stage on every tile shape the launcher picks.

* The config-2 decode sweep (RWKV-7 1.5B: 24 layers x r/k/v/o, ffn_key,
  ffn_value + head, 145 problems, 4-bit g64) as bench.py builds it -- same
  GPU seeds, same GroupedQmv, one planned launch -- at M = 1
  (qmv_stream_table, the headline kernel, including the K = 8192 rows whose
  (scale, bias) windows span four 64-B windows) and M = 8 (qmv_wide_table):
  every output row against the oracle's exact-weight product.
* The config-5 sweep (RWKV-7 7.2B: 32 layers of 3-bit g64 projections at
  K = 4096 / 16384, one planned launch) and its 8-bit head (a second one).
* rq_qmm_lora on the 256 x 128, 128 x 160, 64 x 96 and 8-bit forward tiles
  and on the transposed kernel, with group sizes 32, 64 and 128, against an
  fp32 dense product of the (bit-exact) dequantized weights plus the term.
"""
import pytest
import torch

import bench
from test_gpu_parity import _gpu_dense_ref, acts, bits_equal, rel_check, say, weights

pytestmark = pytest.mark.gpu


def _oracle_rows(O, x, wq, s, b, gs, bits):
    return O.quantized_matmul(x.cpu(), wq.cpu(), s.cpu(), b.cpu(), True, gs, bits,
                              out_dtype=torch.float32, weights="exact")


@pytest.mark.parametrize("M", [1, 8])
def test_config2_benchmarked_plan(O, rq, dev, M):
    say(f"config2 benchmarked plan M={M}: building the 145 problems")
    probs, _ = bench.make_sweep(rq, torch, dev, M=M, timed=False)
    assert len(probs) == bench.LAYERS * len(bench.PROJ) + 1
    xs = [x for _, x, _ in probs]
    ws = [w for _, _, w in probs]
    plan = rq.GroupedQmv(xs, ws, 64, 4)
    assert plan.plan is not None, "the sweep must run as one planned launch"
    say(f"config2 benchmarked plan M={M}: run")
    ys = [y.clone() for y in plan.run()]
    x0 = [x.clone() for x in xs]
    torch.cuda.synchronize()
    # a second run with new activations in the same buffers (as the bench's steps do)
    for i, x in enumerate(xs):
        x.copy_(acts(M, x.shape[-1], 2_500_000 + i).to(dev))
    ys2 = [y.clone() for y in plan.run()]
    torch.cuda.synchronize()
    for i, ((name, x, (wq, s, b)), y, y2) in enumerate(zip(probs, ys, ys2)):
        if i % 24 == 0:
            say(f"config2 M={M}: problem {i} ({name}, {tuple(wq.shape)})")
        ref2 = _oracle_rows(O, x, wq, s, b, 64, 4)
        rel_check(y2, ref2, what=f"config2 M={M} problem {i} {name} rerun")
    for i, ((name, _, (wq, s, b)), x, y) in enumerate(zip(probs, x0, ys)):
        rel_check(y, _oracle_rows(O, x, wq, s, b, 64, 4), what=f"config2 M={M} problem {i} {name}")


def test_config5_benchmarked_plans(O, rq, dev):
    say("config5 benchmarked plans: building 192 3-bit problems + 8-bit head")
    ws, xs, head, xh, _ = bench.config5_sweep(torch, rq, dev)
    p3 = rq.GroupedQmv(xs, ws, 64, 3)
    p8 = rq.GroupedQmv([xh], [head], 64, 8)
    assert p3.plan is not None and p8.plan is not None
    say("config5 benchmarked plans: run")
    ys = p3.run()
    yh = p8.run()[0]
    torch.cuda.synchronize()
    for i, (x, (wq, s, b), y) in enumerate(zip(xs, ws, ys)):
        if i % 32 == 0:
            say(f"config5 problem {i} {tuple(wq.shape)}")
        rel_check(y, _oracle_rows(O, x, wq, s, b, 64, 3), what=f"config5 3-bit problem {i}")
    say("config5 8-bit head")
    rel_check(yh, _oracle_rows(O, xh, *head, 64, 8), what="config5 8-bit head")


# ------------------------------------------------- fused low-rank term

# (transpose, M, R, K, bits, gs): the tile each one runs on
LORA_TILES = [
    (True, 4096, 2048, 2048, 4, 64),    # 256 x 128 (config 4 r/k/v/o forward)
    (True, 4096, 8192, 2048, 4, 64),    # 256 x 128 (config 4 ffn_key forward)
    (True, 2048, 2560, 2560, 4, 64),    # 128 x 160
    (True, 4000, 2560, 1024, 4, 128),   # 256 x 160, gs 128, partial row tile
    (True, 512, 2560, 1024, 4, 32),     # 64 x 96, gs 32, partial column tile
    (True, 1024, 512, 1024, 8, 64),     # 8-bit, 128 x 128
    (True, 4096, 2048, 2048, 8, 128),   # 8-bit, 256 x 128, gs 128
    (False, 4096, 2048, 2048, 4, 64),   # config 4 dX, r/k/v/o
    (False, 4096, 2048, 8192, 4, 64),   # config 4 dX, ffn_value
    (False, 1000, 512, 1024, 8, 128),   # 8-bit transposed, gs 128, partial row tile
    (False, 600, 256, 2048, 4, 32),     # gs 32
    (False, 4096, 2560, 2560, 4, 64),   # transposed, 160-column tiles (2.9B dX)
    (False, 300, 128, 480, 8, 32),      # transposed, 160-column tiles, 8-bit, partial row tile
]


@pytest.mark.parametrize("rank", [16, 64])
@pytest.mark.parametrize("transpose,M,R,K,bits,gs", LORA_TILES)
def test_qmm_lora_every_tile(rq, dev, transpose, M, R, K, bits, gs, rank):
    from rwkvq import ops
    say(f"qmm_lora tiles t={transpose} M={M} R={R} K={K} b={bits} gs={gs} rank={rank}")
    wq, s, b = rq.quantize(weights(R, K, 90_000 + R + K + bits).to(dev), gs, bits)
    n_in, n_out = (K, R) if transpose else (R, K)
    g = torch.Generator().manual_seed(M + rank)
    x = acts(M, n_in, M + R).to(dev)
    z = torch.randn(M, rank, generator=g).to(torch.bfloat16).to(dev)
    L = (torch.randn(n_out, rank, generator=g) * 0.05).to(torch.bfloat16).to(dev)
    y = ops._qmm_lora_fused(x, wq, s, b, z, L, 0.75, transpose, gs, bits)
    assert y is not None, "this problem must run on a 64-wide-stage GEMM"
    ref = _gpu_dense_ref(rq, x, wq, s, b, gs, bits, transpose) + 0.75 * (z.float() @ L.float().t())
    # the term is ~15 % of y here: dropping it, or a wrong scale, fails the bar
    rel_check(y, ref, what=f"qmm_lora t{transpose} {M}x{R}x{K} b{bits} g{gs} r{rank}")


# ----------------------------------------------------- requantize merge

def test_merge_lora_requantize(O, rq, dev):
    """merge_lora(requantize=True) on a QLoRA model: each merged layer is
    QuantizedLinear.from_linear of bf16(dequantize(base) + scale * B A) --
    that merged weight within one bf16 rounding of the oracle's float64 sum,
    its codes, scales and biases bit-exact to the oracle's quantize of it --
    and the merged model's output within quantization error of the adapted
    one."""
    from torch import nn

    class Blk(nn.Module):
        def __init__(self, d, f):
            super().__init__()
            self.tmix = nn.Module()
            for n in ("r_proj", "k_proj", "v_proj", "o_proj"):
                setattr(self.tmix, n, nn.Linear(d, d, bias=False))
            self.cmix = nn.Module()
            self.cmix.key = nn.Linear(d, f, bias=False)
            self.cmix.value = nn.Linear(f, d, bias=False)

    class Model(nn.Module):
        def __init__(self, d=256, f=1024, n=2):
            super().__init__()
            self.blocks = nn.ModuleList(Blk(d, f) for _ in range(n))

    torch.manual_seed(3)
    model = Model().to(dev, torch.bfloat16)
    with torch.no_grad():
        for i, p in enumerate(model.parameters()):
            p.copy_(weights(*p.shape, 31_000 + i).to(dev))
    model, info = rq.add_lora(model, rank=16, alpha=32.0, quantize_base=4, q_group_size=64,
                              cmix_targets=("key", "value"))
    assert info["num_adapters"] == 12
    g = torch.Generator().manual_seed(17)
    with torch.no_grad():
        for m in model.modules():
            if isinstance(m, rq.LoRALinear):
                m.lora_b.copy_((torch.randn(*m.lora_b.shape, generator=g) * 0.02).to(torch.bfloat16))
    x = acts(40, 256, 5).to(dev)
    y_adapted = model.blocks[1].tmix.k_proj(x).float()

    def targets():
        for bi, blk in enumerate(model.blocks):
            for n in ("r_proj", "k_proj", "v_proj", "o_proj"):
                yield bi, blk.tmix, n
            for n in ("key", "value"):
                yield bi, blk.cmix, n

    merged_in = {}
    for bi, parent, name in targets():
        layer = getattr(parent, name)
        wd = O.dequantize(layer.linear.weight.cpu(), layer.linear.scales.cpu(),
                          layer.linear.biases.cpu(), 64, 4).double()
        B, A = layer.lora_b.detach().cpu().double(), layer.lora_a.detach().cpu().double()
        delta = layer.scale * (B @ A)
        exact = wd + delta
        wm = layer.merged_weight(requantize=True).detach().cpu()
        assert wm.dtype == torch.bfloat16
        # one bf16 rounding of an fp32 sum: within a bf16 ulp of the float64
        # value, plus the fp32 errors of the sum and of the rank-16 product
        # B A where the two terms cancel
        bound = (torch.finfo(torch.bfloat16).eps * exact.abs()
                 + 2.0 ** -22 * (wd.abs() + delta.abs())
                 + 2.0 ** -18 * layer.scale * (B.abs() @ A.abs()))
        assert bool(((wm.double() - exact).abs() <= bound).all()), f"block {bi} {name}"
        merged_in[(bi, name)] = wm
        if (bi, name) == (1, "k_proj"):
            expect_k = exact
    with pytest.raises(ValueError):
        rq.merge_lora(model)   # a quantized base needs requantize=True ...
    assert all(isinstance(getattr(p, n), rq.LoRALinear) for _, p, n in targets()), \
        "a refused merge must leave every layer unmerged"
    say("merge_lora requantize")
    rq.merge_lora(model, requantize=True)
    for bi, parent, name in targets():
        q = getattr(parent, name)
        assert isinstance(q, rq.QuantizedLinear) and (q.bits, q.group_size) == (4, 64)
        wq_o, s_o, b_o = O.quantize(merged_in[(bi, name)], 64, 4)
        assert torch.equal(q.weight.cpu(), wq_o), f"block {bi} {name}: codes"
        assert bits_equal(q.scales, s_o) and bits_equal(q.biases, b_o), f"block {bi} {name}"
    # requantizing is not the identity (rwkv_metal/lora/rwkvq_native.py:9-13): the merged
    # layer's output sits at 4-bit g64 quantization error from the dense merged
    # weight's, like any freshly quantized layer (~9 % on N(0, 0.02) weights)
    y_merged = model.blocks[1].tmix.k_proj(x).float()
    y_dense = x.float() @ expect_k.to(dev).float().t()
    err = ((y_merged - y_dense).norm() / y_dense.norm()).item()
    err_adapted = ((y_adapted - y_dense).norm() / y_dense.norm()).item()
    say(f"merged layer vs dense merged weight: {err:.3f}; adapted layer: {err_adapted:.3f}")
    assert err < 0.15 and err_adapted < 0.15

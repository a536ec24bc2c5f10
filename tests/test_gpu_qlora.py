"""GPU parity of the QLoRA layer's kernels (rwkv_metal/lora/lora.py:58-63 under
nn.value_and_grad, rwkv_metal/lora/finetune.py:141): the adapter-gradient
launch rq_lora_grads against fp32 products of the same bf16 operands, and the
whole layer step at BASELINE config 4's full size against an fp32 dense
reference on the dequantized base."""
import pytest
import torch

from test_gpu_parity import acts, rel_check, say, weights

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

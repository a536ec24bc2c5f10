"""Host logic of the Python API without a GPU: argument checks, shape and
dtype inference (meta tensors), module swapping by path predicate, LoRA
wiring, and the refusal to run compute anywhere but the GPU."""
import pytest
import torch
from torch import nn

from rwkv_layout import Tiny  # the reference model's module layout


def test_ops_refuse_cpu_tensors(rq):
    w = torch.randn(8, 64)
    with pytest.raises(RuntimeError, match="GPU"):
        rq.quantize(w, 64, 4)
    wq = torch.zeros(8, 8, dtype=torch.int32)
    s = torch.zeros(8, 1)
    with pytest.raises(RuntimeError, match="GPU"):
        rq.quantized_matmul(torch.randn(2, 64), wq, s, s, True, 64, 4)
    with pytest.raises(RuntimeError, match="GPU"):
        rq.dequantize(wq, s, s, 64, 4)


def test_ops_refuse_operands_on_two_devices():
    from types import SimpleNamespace
    from rwkvq import ops
    on = lambda d: SimpleNamespace(device=torch.device(d))  # only .device is read
    ops._on_gpu(on("cuda:0"), on("cuda:0"))
    with pytest.raises(ValueError, match="one device"):
        ops._on_gpu(on("cuda:0"), on("cuda:0"), on("cuda:1"))
    with pytest.raises(RuntimeError, match="GPU"):
        ops._on_gpu(on("cuda:0"), on("cpu"))


def test_argument_validation(rq):
    w = torch.empty(8, 64, device="meta")
    with pytest.raises(ValueError):
        rq.quantize(w, 64, 7)
    with pytest.raises(ValueError):
        rq.quantize(w, 48, 4)
    with pytest.raises(ValueError):
        rq.quantize(torch.empty(8, 96, device="meta"), 64, 4)
    wq = torch.empty(8, 8, dtype=torch.int32, device="meta")
    s = torch.empty(8, 1, device="meta")
    with pytest.raises(ValueError, match="inner dimension"):
        rq.quantized_matmul(torch.empty(2, 32, device="meta"), wq, s, s, True, 64, 4)
    with pytest.raises(ValueError, match="scales"):
        rq.quantized_matmul(torch.empty(2, 64, device="meta"), wq, s[:4], s[:4], True, 64, 4)


@pytest.mark.parametrize("bits,gs", [(4, 64), (3, 64), (8, 32), (6, 128)])
def test_meta_shapes_and_promotion(rq, bits, gs):
    w = torch.empty(96, 256, device="meta", dtype=torch.bfloat16)
    wq, s, b = rq.quantize(w, gs, bits)
    assert wq.shape == (96, 256 * bits // 32) and wq.dtype == torch.int32
    assert s.shape == b.shape == (96, 256 // gs) and s.dtype == torch.bfloat16
    x = torch.empty(3, 5, 256, device="meta", dtype=torch.bfloat16)
    y = rq.quantized_matmul(x, wq, s, b, True, gs, bits)
    assert y.shape == (3, 5, 96) and y.dtype == torch.bfloat16
    y32 = rq.quantized_matmul(x.float(), wq, s, b, True, gs, bits)
    assert y32.dtype == torch.float32            # MLX promotion: f32 x bf16 -> f32
    dy = torch.empty(7, 96, device="meta", dtype=torch.bfloat16)
    assert rq.quantized_matmul(dy, wq, s, b, False, gs, bits).shape == (7, 256)
    assert rq.dequantize(wq, s, b, gs, bits).shape == (96, 256)


def test_quantize_base_model_selects_big_targets(rq):
    m = Tiny()
    rq.quantize_base_model(m, bits=4, group_size=64)
    assert isinstance(m.head, rq.QuantizedLinear)
    assert isinstance(m.emb, rq.QuantizedEmbedding)
    for blk in m.blocks:
        assert isinstance(blk.cmix.key, rq.QuantizedLinear)
        assert isinstance(blk.cmix.value, rq.QuantizedLinear)
        assert isinstance(blk.tmix.r_proj, nn.Linear)      # left for add_lora
        assert isinstance(blk.tmix.w_lora, nn.Linear)      # low-rank: never quantized
    assert m.blocks[0].cmix.value.weight.shape == (128, 512 * 4 // 32)
    sd = m.state_dict()
    assert {"head.weight", "head.scales", "head.biases"} <= set(sd)


def test_mixed_bits_predicate(rq):
    m = Tiny()
    rq.quantize_model(m, group_size=64, bits=3, class_predicate=lambda p, mod: (
        {"bits": 8} if p == "head" else (rq.is_quantizable(mod) and p.endswith(("key", "value")))))
    assert m.head.bits == 8 and m.blocks[1].cmix.key.bits == 3
    assert isinstance(m.emb, nn.Embedding)


def test_add_lora_wiring_and_freeze(rq):
    m = Tiny()
    rq.quantize_base_model(m, bits=4)
    m, info = rq.add_lora(m, rank=16, alpha=16.0, quantize_base=4, layers=range(1, 3))
    assert info["wrapped_per_block"] == ["tmix.k_proj", "tmix.o_proj", "tmix.r_proj",
                                         "tmix.v_proj"]
    assert info["num_adapters"] == 8
    assert isinstance(m.blocks[0].tmix.r_proj, nn.Linear)
    lora = m.blocks[2].tmix.v_proj
    assert isinstance(lora, rq.LoRALinear) and isinstance(lora.linear, rq.QuantizedLinear)
    assert lora.scale == 1.0 and lora.lora_a.shape == (16, 128) and lora.lora_b.shape == (128, 16)
    trainable = {k for k, p in m.named_parameters() if p.requires_grad}
    assert trainable and all(k.endswith(("lora_a", "lora_b")) for k in trainable)
    assert len(trainable) == 16
    with pytest.raises(ValueError, match="requantize"):
        lora.merged_weight()


def test_negative_layer_indices(rq):
    m = Tiny()
    m, info = rq.add_lora(m, layers=[-1])
    assert isinstance(m.blocks[2].tmix.r_proj, rq.LoRALinear)
    assert not isinstance(m.blocks[0].tmix.r_proj, rq.LoRALinear)


def test_merge_lora_dense_base_cpu(rq):
    torch.manual_seed(0)
    m = Tiny(device="cpu").float()
    m, _ = rq.add_lora(m, rank=4, alpha=8.0, layers=[0])
    lora = m.blocks[0].tmix.r_proj
    with torch.no_grad():
        lora.lora_b.normal_()
    x = torch.randn(3, 128)
    y = lora(x)
    rq.merge_lora(m)
    assert isinstance(m.blocks[0].tmix.r_proj, nn.Linear)
    assert torch.allclose(m.blocks[0].tmix.r_proj(x), y, atol=1e-4, rtol=1e-4)


def test_merge_lora_refuses_quantized_bases_before_merging_anything(rq):
    """Without requantize=True a model with any quantized base raises and no
    layer is merged, including dense-base ones earlier in the module order."""
    m = Tiny(device="cpu").float()
    m, _ = rq.add_lora(m, rank=4, layers=[0, 2])
    blk = m.blocks[2].tmix
    q = rq.QuantizedLinear(128, 128, bias=False, group_size=64, bits=4)
    blk.v_proj = rq.LoRALinear(rank=4, alpha=8.0, base_module=q)
    before = m.blocks[0].tmix.r_proj.linear.weight.clone()
    with pytest.raises(ValueError, match="requantize"):
        rq.merge_lora(m)
    assert all(isinstance(getattr(b.tmix, n), rq.LoRALinear)
               for b in (m.blocks[0], m.blocks[2]) for n in ("r_proj", "k_proj", "v_proj", "o_proj"))
    assert torch.equal(m.blocks[0].tmix.r_proj.linear.weight, before)


def test_save_load_lora_roundtrip(rq, tmp_path):
    torch.manual_seed(1)
    m = Tiny(device="cpu").float()
    m, _ = rq.add_lora(m, rank=4, layers=[1])
    with torch.no_grad():
        m.blocks[1].tmix.k_proj.lora_b.normal_()
    path = str(tmp_path / "adapters.safetensors")
    rq.save_lora(m, path)
    m2 = Tiny(device="cpu").float()
    m2, _ = rq.add_lora(m2, rank=4, layers=[1])
    rq.load_lora(m2, path)
    for k, v in rq.lora_state(m).items():
        assert torch.equal(v, dict(m2.named_parameters())[k])


def _fill_quantized(model, gen):
    """Random packed contents for every quantized module (host only)."""
    for _, m in model.named_modules():
        if isinstance(m, (__import__("rwkvq").QuantizedLinear, __import__("rwkvq").QuantizedEmbedding)):
            m.weight.copy_(torch.randint(-2**31, 2**31 - 1, m.weight.shape, generator=gen,
                                         dtype=torch.int64).to(torch.int32))
            m.scales.copy_(torch.randn(m.scales.shape, generator=gen).to(m.scales.dtype))
            m.biases.copy_(torch.randn(m.biases.shape, generator=gen).to(m.biases.dtype))


def _empty_quantize(rq, model, targets, bits_for):
    """Structure-only quantization (no kernels): swap the targets for empty
    quantized modules of the given bits, group size 64."""
    for path, m in list(model.named_modules()):
        if not any(path.endswith(t) for t in targets):
            continue
        parent_path, _, name = path.rpartition(".")
        parent = model.get_submodule(parent_path) if parent_path else model
        b = bits_for(path)
        if isinstance(m, nn.Linear):
            q = rq.QuantizedLinear(m.in_features, m.out_features, bias=m.bias is not None,
                                   group_size=64, bits=b)
        else:
            q = rq.QuantizedEmbedding(m.num_embeddings, m.embedding_dim, group_size=64, bits=b)
        setattr(parent, name, q)


def test_quantized_checkpoint_roundtrip(rq, tmp_path):
    """save_quantized writes MLX's key names with uint32 packed words and the
    quantization entry (per-module override for the 8-bit head);
    load_quantized rebuilds the quantized modules from shapes alone."""
    from safetensors import safe_open
    from rwkvq import io as rio

    src = Tiny(device="cpu")
    _empty_quantize(rq, src, ("cmix.key", "cmix.value", "head", "emb"),
                    lambda p: 8 if p == "head" else 3)
    g = torch.Generator().manual_seed(5)
    with torch.no_grad():
        _fill_quantized(src, g)
        for p in src.parameters():
            p.copy_(torch.randn(p.shape, generator=g).to(p.dtype))
    path = str(tmp_path / "q.safetensors")
    rio.save_quantized(src, path)
    with safe_open(path, "pt") as f:
        keys = set(f.keys())
        assert f.get_tensor("blocks.0.cmix.key.weight").dtype == torch.uint32
        assert f.get_tensor("head.scales").dtype == torch.bfloat16
    assert {"head.weight", "head.scales", "head.biases", "emb.weight", "emb.scales",
            "blocks.2.cmix.value.biases", "blocks.1.tmix.r_proj.weight"} <= keys
    cfg = rio.quantization_config(path)
    assert cfg["bits"] == 3 and cfg["group_size"] == 64 and cfg["head"] == {"group_size": 64, "bits": 8}

    dst = Tiny(device="cpu")
    rio.load_quantized(dst, path)
    assert isinstance(dst.head, rq.QuantizedLinear) and dst.head.bits == 8
    assert isinstance(dst.emb, rq.QuantizedEmbedding) and dst.emb.bits == 3
    assert isinstance(dst.blocks[1].cmix.value, rq.QuantizedLinear)
    assert dst.blocks[1].cmix.value.bits == 3 and dst.blocks[1].cmix.value.group_size == 64
    assert isinstance(dst.blocks[1].tmix.r_proj, nn.Linear)
    for (k, a), (k2, b) in zip(sorted(src.state_dict().items()), sorted(dst.state_dict().items())):
        assert k == k2 and a.dtype == b.dtype and torch.equal(a, b), k


def test_quantized_checkpoint_mismatch_raises(rq, tmp_path):
    from rwkvq import io as rio
    src = Tiny(device="cpu")
    _empty_quantize(rq, src, ("head",), lambda p: 4)
    path = str(tmp_path / "q.safetensors")
    rio.save_quantized(src, path)
    other = Tiny(d=128, n=2, device="cpu")   # one block fewer: unexpected keys
    with pytest.raises(KeyError):
        rio.load_quantized(other, path)
    rio.load_quantized(Tiny(d=128, n=2, device="cpu"), path, strict=False)


def test_embedding_op_refuses_cpu_and_bad_indices(rq):
    wq = torch.zeros(8, 8, dtype=torch.int32)
    s = torch.zeros(8, 1)
    with pytest.raises(RuntimeError, match="GPU"):
        rq.quantized_embedding(torch.zeros(3, dtype=torch.int64), wq, s, s, 64, 4)
    with pytest.raises(ValueError):
        rq.quantized_embedding(torch.zeros(3), wq, s, s, 64, 4)


@pytest.mark.parametrize("rank,dt", [(16, torch.bfloat16), (8, torch.bfloat16), (16, torch.float16)])
def test_lora_grads_refuses_cpu_tensors(rq, rank, dt):
    """The adapter gradients run on the GPU only, also for the ranks and
    dtypes that take the fp32-product route there: CPU tensors are refused,
    never computed on the host."""
    from rwkvq import ops
    x = torch.zeros(64, 128, dtype=dt)
    u = torch.zeros(64, rank, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU"):
        ops.lora_grads(x, u, x, u, 1.0)
    with pytest.raises(RuntimeError, match="GPU"):
        ops.lora_grads(None, None, x, u, 1.0)

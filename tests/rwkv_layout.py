"""A miniature of the reference model's module layout, shared by the CPU and
GPU tests of quantize_base_model, add_lora and packed checkpoints.

Module paths follow rwkv_metal/model/rwkv7_x070.py: `emb`, `blocks.<i>.tmix.
{r,k,v,o}_proj` (plus low-rank branches such as `w_lora` that are never
quantized, rwkv_metal/lora/finetune.py:40-41), `blocks.<i>.cmix.{key,value}`
and `head`.
"""
import torch
from torch import nn


class TMix(nn.Module):
    def __init__(self, d):
        super().__init__()
        self.r_proj, self.k_proj = nn.Linear(d, d, bias=False), nn.Linear(d, d, bias=False)
        self.v_proj, self.o_proj = nn.Linear(d, d, bias=False), nn.Linear(d, d, bias=False)
        self.w_lora = nn.Linear(d, 32, bias=False)   # low-rank branch, never quantized


class CMix(nn.Module):
    def __init__(self, d):
        super().__init__()
        self.key, self.value = nn.Linear(d, 4 * d, bias=False), nn.Linear(4 * d, d, bias=False)


class Block(nn.Module):
    def __init__(self, d):
        super().__init__()
        self.tmix, self.cmix = TMix(d), CMix(d)


class Tiny(nn.Module):
    """`n` blocks of width `d` with a `vocab`-row embedding and head, in bf16.
    With `seed` set, every weight is drawn from N(0, 0.02) on the CPU
    generator (the embedding from N(0, 1)), then moved to `device`."""

    def __init__(self, d=128, n=3, vocab=256, device="meta", seed=None):
        super().__init__()
        build_on = "cpu" if seed is not None else device
        with torch.device(build_on):
            self.emb = nn.Embedding(vocab, d)
            self.blocks = nn.ModuleList([Block(d) for _ in range(n)])
            self.head = nn.Linear(d, vocab, bias=False)
        if seed is not None:
            g = torch.Generator().manual_seed(seed)
            with torch.no_grad():
                for name, p in self.named_parameters():
                    std = 1.0 if name.startswith("emb") else 0.02
                    p.copy_(torch.randn(p.shape, generator=g) * std)
        self.to(device=device, dtype=torch.bfloat16)

    def forward_parts(self, idx):
        """Every quantizable product the tests compare, keyed by module path."""
        h = self.emb(idx)
        out = {"emb": h}
        for i, blk in enumerate(self.blocks):
            k = blk.cmix.key(h)
            out[f"blocks.{i}.cmix.key"] = k
            out[f"blocks.{i}.cmix.value"] = blk.cmix.value(k)
        out["head"] = self.head(h)
        return out

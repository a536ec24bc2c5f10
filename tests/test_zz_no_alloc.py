"""rq_lora_grads_noalloc (the adapter-gradient launch with its counters and
partial tiles in a static device buffer instead of a workspace) against
rq_lora_grads with a caller workspace, through the C ABI: two calls in a
row, the second with a smaller problem that lays its tiles out differently,
bit for bit, and both within the fp32 bar."""
import pytest
import torch

from test_gpu_parity import rel_check, say

pytestmark = pytest.mark.gpu


def _operands(dev, M, K, N, rank, seed):
    g = torch.Generator().manual_seed(seed)
    mk = lambda *s: torch.randn(*s, generator=g).to(torch.bfloat16).to(dev)  # noqa: E731
    return mk(M, K), mk(M, rank), mk(M, N), mk(M, rank)


def _call(L, fn_name, x, u, dy, z, scale, ws=None):
    from rwkvq.ops import _stream_on
    M, K = x.shape
    N, rank = dy.shape[1], u.shape[1]
    da = torch.full((rank, K), float("nan"), dtype=torch.bfloat16, device=x.device)
    db = torch.full((N, rank), float("nan"), dtype=torch.bfloat16, device=x.device)
    args = [x.data_ptr(), u.data_ptr(), dy.data_ptr(), z.data_ptr(), M, K, N, rank, scale,
            da.data_ptr(), db.data_ptr()]
    if fn_name == "rq_lora_grads":
        args += [ws.data_ptr() if ws is not None else 0, ws.numel() if ws is not None else 0]
    rc = getattr(L, fn_name)(*args, _stream_on(x.device))
    assert rc == 0, L.rq_last_error().decode()
    return da, db


def test_lora_grads_noalloc_matches_workspace_form(rq, dev):
    from rwkvq._lib import lib
    L = lib()
    # the second problem is smaller and has fewer tiles per row chunk
    for M, K, N, rank, seed in [(4096, 2048, 8192, 16, 1), (1000, 520, 136, 32, 2)]:
        say(f"no-alloc lora_grads M={M} K={K} N={N} rank={rank}")
        x, u, dy, z = _operands(dev, M, K, N, rank, seed)
        nbytes = L.rq_lora_grads_workspace_bytes(M, K, N, rank, 1, 1)
        assert nbytes > 0, "the problem must split its rows (the scratch path)"
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
        da_w, db_w = _call(L, "rq_lora_grads", x, u, dy, z, 0.5, ws)
        da_s, db_s = _call(L, "rq_lora_grads_noalloc", x, u, dy, z, 0.5)
        torch.cuda.synchronize()
        assert torch.equal(da_s.view(torch.int16), da_w.view(torch.int16)), "dA differs"
        assert torch.equal(db_s.view(torch.int16), db_w.view(torch.int16)), "dB differs"
        rel_check(da_s, 0.5 * (u.float().t() @ x.float()), what="dA")
        rel_check(db_s, 0.5 * (dy.float().t() @ z.float()), what="dB")

"""rq_lora_grads_noalloc (the adapter-gradient launch with its counters and
partial tiles in a static device buffer instead of a workspace) against
rq_lora_grads with a caller workspace, through the C ABI: two calls in a
row, the second with a smaller problem that lays its tiles out differently,
bit for bit, and both within the fp32 bar; and the same call captured into a
HIP graph (the callers this entry point is for), replayed several times with
eager calls between the replays.  The graph test comes first in the file so
that, in a fresh process, it also covers the first call on the device being
made under capture."""
import pytest
import torch

from test_gpu_parity import rel_check, say

pytestmark = pytest.mark.gpu


def _operands(dev, M, K, N, rank, seed):
    g = torch.Generator().manual_seed(seed)
    mk = lambda *s: torch.randn(*s, generator=g).to(torch.bfloat16).to(dev)  # noqa: E731
    return mk(M, K), mk(M, rank), mk(M, N), mk(M, rank)


def _call(L, fn_name, x, u, dy, z, scale, ws=None, out=None):
    from rwkvq.ops import _stream_on
    M, K = x.shape
    N, rank = dy.shape[1], u.shape[1]
    if out is None:
        da = torch.full((rank, K), float("nan"), dtype=torch.bfloat16, device=x.device)
        db = torch.full((N, rank), float("nan"), dtype=torch.bfloat16, device=x.device)
    else:
        da, db = out
    args = [x.data_ptr(), u.data_ptr(), dy.data_ptr(), z.data_ptr(), M, K, N, rank, scale,
            da.data_ptr(), db.data_ptr()]
    if fn_name == "rq_lora_grads":
        args += [ws.data_ptr() if ws is not None else 0, ws.numel() if ws is not None else 0]
    rc = getattr(L, fn_name)(*args, _stream_on(x.device))
    assert rc == 0, L.rq_last_error().decode()
    return da, db


def test_lora_grads_noalloc_in_a_hip_graph(rq, dev):
    from rwkvq._lib import lib
    L = lib()
    M, K, N, rank = 4096, 2048, 2048, 16
    say(f"no-alloc lora_grads under graph capture M={M} K={K} N={N} rank={rank}")
    x, u, dy, z = _operands(dev, M, K, N, rank, 5)
    nbytes = L.rq_lora_grads_workspace_bytes(M, K, N, rank, 1, 1)
    assert nbytes > 0, "the problem must split its rows (the scratch path)"
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    da_w, db_w = _call(L, "rq_lora_grads", x, u, dy, z, 0.25, ws)
    out = (torch.full((rank, K), float("nan"), dtype=torch.bfloat16, device=dev),
           torch.full((N, rank), float("nan"), dtype=torch.bfloat16, device=dev))
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _call(L, "rq_lora_grads_noalloc", x, u, dy, z, 0.25, out=out)
    torch.cuda.synchronize()
    small = _operands(dev, 1000, 520, 136, 32, 6)
    for replay in range(3):
        out[0].fill_(float("nan"))
        out[1].fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out[0].view(torch.int16), da_w.view(torch.int16)), f"dA, replay {replay}"
        assert torch.equal(out[1].view(torch.int16), db_w.view(torch.int16)), f"dB, replay {replay}"
        # an eager call on the same scratch between replays, checked as well
        da_e, db_e = _call(L, "rq_lora_grads_noalloc", *small, 0.5)
        torch.cuda.synchronize()
        rel_check(da_e, 0.5 * (small[1].float().t() @ small[0].float()), what="eager dA")
        rel_check(db_e, 0.5 * (small[2].float().t() @ small[3].float()), what="eager dB")
    rel_check(out[0], 0.25 * (u.float().t() @ x.float()), what="graph dA")
    rel_check(out[1], 0.25 * (dy.float().t() @ z.float()), what="graph dB")


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

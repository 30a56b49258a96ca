"""moc_chapter_plan_noalloc (the plan on the library's fixed device scratch array, no
allocation) against moc_chapter_plan with a caller workspace: two calls in a row, the second on a
smaller input, both large enough for the multi-kernel path that uses the workspace; outputs are
integer and must be identical.  A plan larger than the scratch array is refused on the host."""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _plan(L, chap, C, noalloc):
    dev = chap.device
    E = chap.numel()
    mu = min(E, C)
    out = [torch.full((mu,), -7, device=dev, dtype=torch.int32), torch.full((2,), -7, device=dev, dtype=torch.int32),
           torch.full((E,), -7, device=dev, dtype=torch.int32), torch.full((mu + 1,), -7, device=dev, dtype=torch.int32),
           torch.full((E,), -7, device=dev, dtype=torch.int32)]
    st = L.stream_ptr(dev)
    if noalloc:
        L.call("moc_chapter_plan_noalloc", L.ptr(chap), E, C, *(L.ptr(t) for t in out), st)
    else:
        ws_bytes = L.query("moc_chapter_plan_workspace", E, C)
        ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
        L.call("moc_chapter_plan", L.ptr(chap), E, C, L.ptr(ws), ws_bytes, *(L.ptr(t) for t in out), st)
        torch.cuda.synchronize()
    return out


def test_noalloc_plan_matches_workspace_plan(gpu_device):
    from memory_amd import _lib as L
    L.lib()
    g = torch.Generator().manual_seed(0)
    for E, C in ((200_000, 4097), (5_000, 1000)):          # the second call smaller than the first
        print(f"noalloc plan E={E} C={C}", flush=True)
        chap = torch.randint(-3, C + 3, (E,), generator=g, dtype=torch.int32)   # a few skipped edges
        chap_d = chap.to(gpu_device)
        got = _plan(L, chap_d, C, True)
        torch.cuda.synchronize()
        want = _plan(L, chap_d, C, False)
        n_u = int(want[1][0])
        assert int(got[1][0]) == n_u and int(got[1][1]) == int(want[1][1])
        assert torch.equal(got[0][:n_u].cpu(), want[0][:n_u].cpu())
        assert torch.equal(got[2].cpu(), want[2].cpu())
        assert torch.equal(got[3][:n_u + 1].cpu(), want[3][:n_u + 1].cpu())
        assert torch.equal(got[4].cpu(), want[4].cpu())
        valid = chap[(chap >= 0) & (chap < C)]
        assert n_u == int(torch.unique(valid).numel())


def test_noalloc_plan_refuses_plans_beyond_the_scratch(gpu_device):
    from memory_amd import _lib as L
    E, C = 1_000_000, 16_384
    assert L.query("moc_chapter_plan_workspace", E, C) > (4 << 20)
    chap = torch.zeros(E, device=gpu_device, dtype=torch.int32)
    dummy = torch.empty(E + C + 2, device=gpu_device, dtype=torch.int32)
    with pytest.raises(ValueError, match="scratch"):
        L.call("moc_chapter_plan_noalloc", L.ptr(chap), E, C, L.ptr(dummy), L.ptr(dummy), L.ptr(dummy), L.ptr(dummy),
               L.ptr(dummy), L.stream_ptr(gpu_device))


def test_noalloc_plan_graph_replay(gpu_device):
    """The entry point captured into a HIP graph after one uncaptured call: every replay, on new
    chapter ids written into the captured input, with eager work and synchronisation between the
    replays, equals moc_chapter_plan on the same ids."""
    from memory_amd import _lib as L
    L.lib()
    g = torch.Generator().manual_seed(1)
    E, C = 150_000, 4097
    chap_d = torch.randint(0, C, (E,), generator=g, dtype=torch.int32).to(gpu_device)
    mu = min(E, C)
    outs = [torch.full((mu,), -7, device=gpu_device, dtype=torch.int32),
            torch.full((2,), -7, device=gpu_device, dtype=torch.int32),
            torch.full((E,), -7, device=gpu_device, dtype=torch.int32),
            torch.full((mu + 1,), -7, device=gpu_device, dtype=torch.int32),
            torch.full((E,), -7, device=gpu_device, dtype=torch.int32)]
    L.call("moc_chapter_plan_noalloc", L.ptr(chap_d), E, C, *(L.ptr(t) for t in outs), L.stream_ptr(gpu_device))
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            L.call("moc_chapter_plan_noalloc", L.ptr(chap_d), E, C, *(L.ptr(t) for t in outs),
                   L.stream_ptr(gpu_device))
    torch.cuda.current_stream().wait_stream(side)
    for rep in range(3):
        lo = -2 if rep == 1 else 0
        chap = torch.randint(lo, C // (rep + 1), (E,), generator=g, dtype=torch.int32)
        chap_d.copy_(chap.to(gpu_device))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in outs]
        want = _plan(L, chap_d, C, False)   # eager plan with its own workspace between the replays
        n_u = int(want[1][0])
        print(f"replay {rep}: E={E} C={C} n_uniq={n_u}", flush=True)
        assert int(got[1][0]) == n_u and int(got[1][1]) == int(want[1][1])
        assert torch.equal(got[0][:n_u].cpu(), want[0][:n_u].cpu())
        assert torch.equal(got[2].cpu(), want[2].cpu())
        assert torch.equal(got[3][:n_u + 1].cpu(), want[3][:n_u + 1].cpu())
        # csr_edge is defined for the valid edges only (csr_off[n_uniq] of them); the captured
        # buffer keeps an earlier replay's entries past them
        tot = int(want[3][n_u])
        assert torch.equal(got[4][:tot].cpu(), want[4][:tot].cpu())

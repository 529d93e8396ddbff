"""Helpers shared by the GPU tests."""
import torch


def graph_replays_match(fn, out_fn, n_replays: int = 3) -> bool:
    """Capture fn() in a hipGraph (torch.cuda.CUDAGraph) after side-stream
    warm-up, replay it n times with eager work and syncs in between, and check
    every replay bitwise against an eager run. out_fn() returns the tensor the
    graph writes."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    eager = out_fn().clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    ok = True
    for _ in range(n_replays):
        out_fn().zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        ok &= torch.equal(out_fn(), eager)
        _ = torch.randn(1024, device="cuda").sum().item()  # unrelated eager work
    return ok

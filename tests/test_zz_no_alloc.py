"""acorn_paged_attention_noalloc, the allocation-free K3 entry point, through
the C-ABI: on two calls in a row (the second smaller) its output equals
acorn_paged_attention's with caller-owned workspaces bit for bit (the same
kernels) and the oracle within the bf16 bar; a request beyond the fixed
scratch is refused with ACORN_ERR_SCRATCH before anything is launched; one
split needs no scratch at any size; after one warm-up call the entry point
records into a hipGraph and every replay equals the workspace entry point."""
import pytest
import torch

from acorninfer_amd import _lib
from acorninfer_amd._lib import dtype_code, lib, ptr, stream_ptr
from oracle.ops_ref import paged_attention_ref
from tolerances import TOL_BF16

H, KV, D, P = 32, 8, 128, 16


def _inputs(B, lo, hi, width, seed):
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(lo, hi + 1, (B,), generator=g, dtype=torch.int32)
    nb = int(sum(-(-int(n) // P) for n in lens)) + 8
    perm = torch.randperm(nb, generator=g).to(torch.int32)
    tables = torch.zeros(B, width, dtype=torch.int32)
    off = 0
    for b in range(B):
        n = -(-int(lens[b]) // P)
        tables[b, :n] = perm[off:off + n]
        off += n
    q = torch.randn(B, H, D, generator=g).bfloat16()
    kp = torch.randn(nb, P, KV, D, generator=g).bfloat16()
    vp = torch.randn(nb, P, KV, D, generator=g).bfloat16()
    return q, kp, vp, tables, lens


def _call(noalloc, q, kp, vp, tables, lens, S, out):
    B = q.shape[0]
    args_a = (ptr(q), ptr(kp), ptr(vp), ptr(tables), ptr(lens), ptr(out))
    args_b = (B, H, KV, D, P, kp.shape[0], tables.shape[1], S, float(D ** -0.5), dtype_code(q),
              stream_ptr(q.device))
    if noalloc:
        return lib().acorn_paged_attention_noalloc(*args_a, *args_b)
    acc = torch.empty(B * H * S * D, dtype=torch.float32, device=q.device)
    ml = torch.empty(2 * B * H * S, dtype=torch.float32, device=q.device)
    return lib().acorn_paged_attention(*args_a, ptr(acc), ptr(ml), *args_b)


@pytest.mark.gpu
def test_noalloc_equals_workspace_entry_on_two_calls_second_smaller():
    cases = [(8, 512, 4096, 256, 64, 1), (3, 20, 900, 64, 16, 2)]   # config 2, then smaller
    for B, lo, hi, width, S, seed in cases:
        print(f"\n[noalloc B={B} ctx {lo}..{hi} width {width} S={S}]", flush=True)
        host = _inputs(B, lo, hi, width, seed)
        q, kp, vp, tables, lens = (t.cuda() for t in host)
        want = torch.empty_like(q)
        got = torch.full_like(q, float("nan"))
        assert _call(False, q, kp, vp, tables, lens, S, want) == 0
        torch.cuda.synchronize()
        # torch's allocator and the device's free memory (a hipMalloc inside
        # the library would show in the second)
        before, free_before = torch.cuda.memory_allocated(), torch.cuda.mem_get_info()[0]
        assert _call(True, q, kp, vp, tables, lens, S, got) == 0
        torch.cuda.synchronize()
        assert torch.cuda.memory_allocated() == before
        assert torch.cuda.mem_get_info()[0] == free_before
        assert torch.equal(got, want)
        torch.testing.assert_close(got.cpu(), paged_attention_ref(*host), **TOL_BF16)


@pytest.mark.gpu
def test_noalloc_refuses_more_than_its_scratch():
    B, S = 64, 64                     # 64*32*64*(128+2) fp32 = 68 MB > 32 MiB
    assert B * H * S * (D + 2) * 4 > _lib.K3_SCRATCH_BYTES
    host = _inputs(B, 1, 64, 4, 3)
    q, kp, vp, tables, lens = (t.cuda() for t in host)
    out = torch.full_like(q, 7.0)
    rc = _call(True, q, kp, vp, tables, lens, S, out)
    assert rc == _lib.ERR_SCRATCH
    with pytest.raises(ValueError, match="scratch"):
        _lib.check(rc, "paged_attention_noalloc")
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())   # nothing was launched
    # one split keeps no partials: any size runs
    assert _call(True, q, kp, vp, tables, lens, 1, out) == 0
    want = torch.empty_like(q)
    assert _call(False, q, kp, vp, tables, lens, 1, want) == 0
    torch.cuda.synchronize()
    assert torch.equal(out, want)


@pytest.mark.gpu
def test_noalloc_graph_capture_replays_bitwise():
    """Captured after one warm-up call (which looks up the scratch address),
    the entry point replays with the same bits as the workspace entry point,
    replay after replay, with eager work and synchronisation in between."""
    B, S = 8, 64
    host = _inputs(B, 512, 4096, 256, 11)
    q, kp, vp, tables, lens = (t.cuda() for t in host)
    want = torch.empty_like(q)
    assert _call(False, q, kp, vp, tables, lens, S, want) == 0
    out = torch.empty_like(q)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        assert _call(True, q, kp, vp, tables, lens, S, out) == 0     # warm-up
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            assert _call(True, q, kp, vp, tables, lens, S, out) == 0
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for rep in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {rep}"

"""Speculative-verify attention (ops/paged_verify.py over K3) and the verify
write path (PagedKVCache.scatter_verify), on the GPU, against the oracle
(oracle.ops_ref.paged_verify_ref, restating acorninfer/ops/paged_verify.py:
96-123; pinned in test_verify_host.py).

Coverage follows the reference's tests/test_paged_verify.py: the matrix
B in {1,4,7} x m in {2,5} x history in {1,15,16,17,48} with ragged batches and
split counts that leave splits empty, at fp32 (TOL_F32) and bf16 (TOL_BF16);
window causality exactly (k = 0 makes every row the mean of its visible v;
poisoned future window rows and NaN slots past the length fail it); and the
rollback path (write a window, roll back, rewrite the dead slots) ending in
the same pages and outputs as a cache that never held them. The Qwen3 shape
(32/8 heads, D = 128) runs the MFMA K3 form."""
import pytest
import torch

from oracle.ops_ref import paged_verify_ref
from tolerances import TOL_BF16, TOL_F32

pytestmark = pytest.mark.gpu

_S_BY_HIST = {1: 4, 15: 2, 16: 1, 17: 4, 48: 8}
MATRIX = [(B, M, h, _S_BY_HIST[h]) for B in (1, 4, 7) for M in (2, 5) for h in _S_BY_HIST]


def _inputs(B, M, hist, dtype, H=4, KV=2, D=16, P=16, seed=8):
    g = torch.Generator().manual_seed(seed)
    lens = [hist + b + M for b in range(B)]
    mp = max(-(-n // P) for n in lens)
    nb = mp + 2
    q = torch.randn(B, M, H, D, generator=g).to(dtype)
    kp = torch.randn(nb, P, KV, D, generator=g).to(dtype)
    vp = torch.randn(nb, P, KV, D, generator=g).to(dtype)
    tables = torch.empty(B, mp, dtype=torch.int32)
    for i, n in enumerate(lens):
        used = -(-n // P)
        tables[i, :used] = torch.randperm(nb, generator=g)[:used]
        tables[i, used:] = torch.randint(0, nb, (mp - used,), generator=g)
    return q, kp, vp, tables, torch.tensor(lens, dtype=torch.int32)


def _gpu(*ts):
    return [t.cuda() for t in ts]


@pytest.mark.parametrize("dtype,tol", [(torch.float32, TOL_F32), (torch.bfloat16, TOL_BF16)])
def test_verify_matrix_matches_oracle(dtype, tol):
    from acorninfer_amd.ops.paged_verify import paged_verify_attention
    for B, M, hist, S in MATRIX:
        q, kp, vp, tables, lens = _inputs(B, M, hist, dtype)
        out = paged_verify_attention(*_gpu(q, kp, vp, tables, lens), S)
        ref = paged_verify_ref(q, kp, vp, tables, lens)
        torch.testing.assert_close(out.cpu().float(), ref.float(), **tol,
                                   msg=f"B={B} m={M} hist={hist} S={S}")


@pytest.mark.parametrize("S", [1, 3, 8])
def test_verify_qwen3_shape_bf16(S):
    from acorninfer_amd.ops.paged_verify import paged_verify_attention
    q, kp, vp, tables, lens = _inputs(4, 4, 100, torch.bfloat16, H=32, KV=8, D=128, seed=5)
    out = paged_verify_attention(*_gpu(q, kp, vp, tables, lens), S)
    ref = paged_verify_ref(q, kp, vp, tables, lens)
    torch.testing.assert_close(out.cpu().float(), ref.float(), **TOL_BF16)


def test_window_of_one_is_decode_bitwise():
    from acorninfer_amd.ops.paged_attention import paged_decode_attention
    from acorninfer_amd.ops.paged_verify import paged_verify_attention
    q, kp, vp, tables, lens = _gpu(*_inputs(3, 1, 40, torch.bfloat16, H=32, KV=8, D=128))
    a = paged_verify_attention(q, kp, vp, tables, lens, 4)[:, 0]
    b = paged_decode_attention(q[:, 0].contiguous(), kp, vp, tables, lens, 4)
    assert torch.equal(a, b)


@pytest.mark.parametrize("dtype,H,KV,D", [(torch.float32, 4, 2, 16), (torch.bfloat16, 32, 8, 128)])
def test_window_causality_exact(dtype, H, KV, D):
    """k = 0: every visible score is 0, so row (b, j) is the plain mean of the
    v of tokens 0 .. hist_b + j. The window's later rows carry v x 100 (a row
    that sees past its position is far off), and every slot past the length
    and the padding page hold NaN (a read past the length shows)."""
    from acorninfer_amd.ops.paged_verify import paged_verify_attention
    g = torch.Generator().manual_seed(11)
    B, M, P = 3, 5, 16
    hist = [8 + b for b in range(B)]
    nb = B + 1
    kp = torch.zeros(nb, P, KV, D)
    vp = torch.zeros(nb, P, KV, D)
    kp[nb - 1] = float("nan")
    vp[nb - 1] = float("nan")
    tables = torch.full((B, 2), nb - 1, dtype=torch.int32)
    dense = []
    for b in range(B):
        tables[b, 0] = b
        L = hist[b] + M
        v = torch.randn(L, KV, D, generator=g)
        v[hist[b] + 1:] *= 100.0
        vp[b, :L] = v
        vp[b, L:] = float("nan")
        kp[b, L:] = float("nan")
        dense.append(v.to(dtype).float())
    lens = torch.tensor([h + M for h in hist], dtype=torch.int32)
    q = torch.randn(B, M, H, D, generator=g)
    out = paged_verify_attention(*_gpu(q.to(dtype), kp.to(dtype), vp.to(dtype), tables, lens), 4)
    out = out.cpu().float()
    assert torch.isfinite(out).all()
    for b in range(B):
        for j in range(M):
            want = dense[b][:hist[b] + j + 1].mean(0)               # [KV, D]
            got = out[b, j].view(KV, H // KV, D)
            for r in range(H // KV):
                torch.testing.assert_close(got[:, r], want, rtol=2e-2 if dtype != torch.float32 else 1e-4,
                                           atol=2e-2 if dtype != torch.float32 else 1e-3)


def test_scatter_verify_bit_exact_and_lengths():
    from acorninfer_amd.cache.pager import BlockAllocator, PagedCacheView, PagedKVCache
    KV, D, P, m = 8, 128, 16, 5
    cache = PagedKVCache(2, KV, D, P, BlockAllocator(16), "cuda", torch.bfloat16)
    views = [PagedCacheView(cache) for _ in range(3)]
    for i, v in enumerate(views):
        for li in range(2):
            v._lens[li] = 13 + 7 * i
    targets = [v.ensure_append_capacity_n(1, m) for v in views]
    pages = torch.tensor([[p for p, _ in t] for t in targets], dtype=torch.long, device="cuda")
    slots = torch.tensor([[s for _, s in t] for t in targets], dtype=torch.long, device="cuda")
    k = torch.randn(3, KV, m, D, device="cuda", dtype=torch.bfloat16)
    v = torch.randn(3, KV, m, D, device="cuda", dtype=torch.bfloat16)
    want_k, want_v = cache.k_pages[1].clone(), cache.v_pages[1].clone()
    want_k[pages.reshape(-1), slots.reshape(-1)] = k.permute(0, 2, 1, 3).reshape(-1, KV, D)
    want_v[pages.reshape(-1), slots.reshape(-1)] = v.permute(0, 2, 1, 3).reshape(-1, KV, D)
    cache.scatter_verify(views, 1, k, v, pages, slots)
    assert torch.equal(cache.k_pages[1], want_k) and torch.equal(cache.v_pages[1], want_v)
    assert [vw._lens[1] for vw in views] == [13 + 7 * i + m for i in range(3)]
    assert [vw._lens[0] for vw in views] == [13 + 7 * i for i in range(3)]


def test_rollback_then_rewrite_equals_a_cache_that_never_held_the_dead_slots():
    """Window of 5 written at 13..17, 2 accepted (length back to 16), the next
    window reuses the dead slots 16, 17 and goes on in the same page: pages
    and verify outputs equal (bitwise) a twin that wrote the surviving tokens
    directly, and the oracle (TOL_F32)."""
    from acorninfer_amd.cache.pager import BlockAllocator, PagedCacheView, PagedKVCache
    from acorninfer_amd.ops.paged_verify import paged_verify_attention
    torch.manual_seed(3)
    KV, D, P, H, m, base, acc = 2, 16, 16, 4, 5, 13, 2
    pre_k, pre_v = torch.randn(1, KV, base, D).cuda(), torch.randn(1, KV, base, D).cuda()
    k1, v1 = torch.randn(1, KV, m, D).cuda(), torch.randn(1, KV, m, D).cuda()
    k2, v2 = torch.randn(1, KV, m, D).cuda(), torch.randn(1, KV, m, D).cuda()

    def make():
        cache = PagedKVCache(1, KV, D, P, BlockAllocator(8), "cuda", torch.float32)
        return cache, PagedCacheView(cache)

    def window(cache, view, k, v):
        t = view.ensure_append_capacity_n(0, m)
        pg = torch.tensor([[p for p, _ in t]], dtype=torch.long, device="cuda")
        sl = torch.tensor([[s for _, s in t]], dtype=torch.long, device="cuda")
        cache.scatter_verify([view], 0, k, v, pg, sl)
        return t

    ca, va = make()
    va.write(0, pre_k, pre_v)
    t1 = window(ca, va, k1, v1)
    assert va.seq_len == base + m and len(va.table) == 2
    va.set_lens(0, base + acc + 1)
    t2 = window(ca, va, k2, v2)
    assert t2[:2] == t1[3:5]                                  # the dead slots are reused
    assert va.seq_len == base + acc + 1 + m

    cb, vb = make()
    vb.write(0, torch.cat([pre_k, k1[:, :, :acc + 1]], 2), torch.cat([pre_v, v1[:, :, :acc + 1]], 2))
    vb.write(0, k2, v2)
    L = va.seq_len
    for pages_a, pages_b in ((ca.k_pages[0], cb.k_pages[0]), (ca.v_pages[0], cb.v_pages[0])):
        ga = pages_a[torch.tensor(va.table, device="cuda")].reshape(-1, KV, D)[:L]
        gb = pages_b[torch.tensor(vb.table, device="cuda")].reshape(-1, KV, D)[:L]
        assert torch.equal(ga, gb)
    q = torch.randn(1, m, H, D).cuda()
    lens = torch.tensor([L], dtype=torch.int32, device="cuda")
    ta = torch.tensor([va.table], dtype=torch.int32, device="cuda")
    tb = torch.tensor([vb.table], dtype=torch.int32, device="cuda")
    oa = paged_verify_attention(q, ca.k_pages[0], ca.v_pages[0], ta, lens, 2)
    ob = paged_verify_attention(q, cb.k_pages[0], cb.v_pages[0], tb, lens, 2)
    assert torch.equal(oa, ob)
    ref = paged_verify_ref(q.cpu(), ca.k_pages[0].cpu(), ca.v_pages[0].cpu(), ta.cpu(), lens.cpu())
    torch.testing.assert_close(oa.cpu(), ref, **TOL_F32)

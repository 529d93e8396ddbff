"""Prefill attention (acorn_paged_prefill_attention, HIP) vs the oracle.

A sequence's run of nq prompt rows from KV position pos0 is a window of
m = nq rows over seq_lens = pos0 + nq tokens: exactly what
oracle/ops_ref.paged_verify_ref restates (acorninfer/ops/paged_verify.py:
96-123, pinned against a float64 brute force over an explicit causal mask),
and row j of it equals the decode oracle paged_attention_ref at length
pos0 + j + 1 (acorninfer/ops/paged_attention.py:192-216), the semantics of
the reference's prefill SDPA (models/qwen3.py:291-382: is_causal for an empty
cache, bottom-right causal for an extension).

Cases: one token; exact 16-token tiles and ragged tails; a chunk continuing
a cached prefix; several packed sequences with uncovered rows left as they
were; GQA 1/2/4/8; D 64/128; pages 16/32; bf16 and fp16. At 8192 tokens
(the long-context serving workload's context) sampled rows against the
oracle and every row against K3, the per-row decode kernel. Also
determinism, graph replay and the row bound.
"""
import pytest
import torch

from oracle.ops_ref import paged_attention_ref, paged_verify_ref
from tolerances import TOL_BF16, max_abs_diff
from gpu_utils import graph_replays_match

# (H, KV, D, P, [(pos0, nq), ...])
CASES = [
    (4, 4, 64, 16, [(0, 1)]),
    (8, 2, 64, 16, [(0, 16)]),
    (32, 8, 128, 16, [(0, 17)]),
    (32, 8, 128, 16, [(0, 100)]),
    (32, 8, 128, 16, [(20, 21)]),
    (16, 8, 128, 32, [(37, 5)]),
    (32, 8, 128, 16, [(0, 5), (0, 33), (10, 17)]),
    (64, 8, 128, 16, [(3, 40), (64, 64)]),
    (8, 8, 128, 16, [(100, 70), (0, 2)]),
    (16, 8, 64, 32, [(0, 65), (31, 1)]),
]


def _make(H, KV, D, P, segs, dtype, seed, gap=3):
    """Pool, per-sequence tables and packed q with `gap` uncovered rows
    between sequences."""
    g = torch.Generator().manual_seed(seed)
    pages = [-(-(p0 + n) // P) for p0, n in segs]
    nb = sum(pages) + 3
    k_pages = torch.randn(nb, P, KV, D, generator=g).to(dtype)
    v_pages = torch.randn(nb, P, KV, D, generator=g).to(dtype)
    W = max(pages)
    perm = torch.randperm(nb, generator=g)
    tables = torch.randint(0, nb, (len(segs), W), generator=g).to(torch.int32)
    used = 0
    for i, n in enumerate(pages):
        tables[i, :n] = perm[used:used + n]
        used += n
    row0, r = [], gap
    for _, n in segs:
        row0.append(r)
        r += n + gap
    q = torch.randn(r, H, D, generator=g).to(dtype)
    meta = (torch.tensor(row0, dtype=torch.int32),
            torch.tensor([p for p, _ in segs], dtype=torch.int32),
            torch.tensor([n for _, n in segs], dtype=torch.int32))
    return q, k_pages, v_pages, tables, meta


def _oracle(q, k_pages, v_pages, tables, meta):
    row0, pos0, nq = meta
    out = {}
    for i in range(len(row0)):
        a, n, p0 = int(row0[i]), int(nq[i]), int(pos0[i])
        win = q[a:a + n][None]                                    # [1, m, H, D]
        out[i] = paged_verify_ref(win, k_pages, v_pages, tables[i][None],
                                  torch.tensor([p0 + n]))[0]
    return out


def _run(q, k_pages, v_pages, tables, meta, out=None):
    from acorninfer_amd.ops.paged_attention import paged_prefill_attention
    row0, pos0, nq = meta
    return paged_prefill_attention(q.cuda(), k_pages.cuda(), v_pages.cuda(), tables.cuda(),
                                   row0.cuda(), pos0.cuda(), nq.cuda(), int(nq.max()), out=out)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prefill_attention_matches_oracle(dtype):
    worst = 0.0
    for ci, (H, KV, D, P, segs) in enumerate(CASES):
        q, kp, vp, tb, meta = _make(H, KV, D, P, segs, dtype, seed=40 + ci)
        print(f"\n[prefill attention case {ci}: H={H} KV={KV} D={D} P={P} segs={segs}]",
              flush=True)
        sentinel = torch.full_like(q, 7.0).cuda()
        got = _run(q, kp, vp, tb, meta, out=sentinel).cpu()
        want = _oracle(q, kp, vp, tb, meta)
        covered = torch.zeros(q.shape[0], dtype=torch.bool)
        row0, _, nq = meta
        for i, w in want.items():
            a, n = int(row0[i]), int(nq[i])
            torch.testing.assert_close(got[a:a + n], w, **TOL_BF16)
            worst = max(worst, max_abs_diff(got[a:a + n], w))
            covered[a:a + n] = True
        assert bool((got[~covered] == 7.0).all()), "rows outside every sequence were written"
    print(f"\n[prefill attention {dtype}: max|diff| vs oracle {worst:.3g}]")


@pytest.mark.gpu
def test_prefill_attention_rows_equal_decode_oracle_rows():
    """Row j of a run is the decode oracle at length pos0 + j + 1 (the
    second, per-row restatement)."""
    H, KV, D, P = 32, 8, 128, 16
    q, kp, vp, tb, meta = _make(H, KV, D, P, [(5, 40)], torch.bfloat16, seed=77, gap=0)
    got = _run(q, kp, vp, tb, meta).cpu()
    lens = torch.arange(6, 46, dtype=torch.int32)
    want = paged_attention_ref(q, kp, vp, tb.expand(40, -1), lens)
    torch.testing.assert_close(got, want, **TOL_BF16)


@pytest.mark.gpu
def test_prefill_attention_8192_tokens_vs_oracle_rows_and_k3():
    """A whole 8192-token prompt (Qwen3-8B heads): sampled rows against the
    oracle, every row against K3 with one decode row per token."""
    from acorninfer_amd.ops.paged_attention import paged_decode_attention
    H, KV, D, P, L = 32, 8, 128, 16, 8192
    q, kp, vp, tb, meta = _make(H, KV, D, P, [(0, L)], torch.bfloat16, seed=91, gap=0)
    print(f"\n[prefill attention: one prompt of {L} tokens]", flush=True)
    got = _run(q, kp, vp, tb, meta).cpu()
    rows = [0, 1, 15, 16, 17, 31, 32, 1000, 4095, 4096, 6143, 8190, 8191]
    want = paged_attention_ref(q[rows], kp, vp, tb.expand(len(rows), -1),
                               torch.tensor([r + 1 for r in rows], dtype=torch.int32))
    torch.testing.assert_close(got[rows], want, **TOL_BF16)
    k3 = paged_decode_attention(q.cuda(), kp.cuda(), vp.cuda(), tb.expand(L, -1).contiguous().cuda(),
                                torch.arange(1, L + 1, dtype=torch.int32).cuda(), 4).cpu()
    torch.testing.assert_close(got, k3, **TOL_BF16)
    print(f"\n[8192-token prefill: max|diff| vs K3 {max_abs_diff(got, k3):.3g}]")


@pytest.mark.gpu
def test_prefill_attention_chunked_equals_whole():
    """A prompt in two chunks (the second continuing the cached first) gives
    the whole prompt's rows: the same keys, the same causal limits."""
    H, KV, D, P = 32, 8, 128, 16
    q, kp, vp, tb, meta = _make(H, KV, D, P, [(0, 300)], torch.bfloat16, seed=5, gap=0)
    whole = _run(q, kp, vp, tb, meta).cpu()
    first = _run(q[:130], kp, vp, tb, (torch.tensor([0], dtype=torch.int32),
                                        torch.tensor([0], dtype=torch.int32),
                                        torch.tensor([130], dtype=torch.int32))).cpu()
    second = _run(q[130:], kp, vp, tb, (torch.tensor([0], dtype=torch.int32),
                                         torch.tensor([130], dtype=torch.int32),
                                         torch.tensor([170], dtype=torch.int32))).cpu()
    # 130 is not a multiple of 16, so the second chunk's rows sit in other
    # query tiles than in the whole run (other rescaling points of the
    # online softmax): equal within the activation tolerance
    torch.testing.assert_close(torch.cat([first, second]), whole, **TOL_BF16)


@pytest.mark.gpu
def test_prefill_attention_deterministic_graph_and_row_bound():
    H, KV, D, P = 32, 8, 128, 16
    q, kp, vp, tb, meta = _make(H, KV, D, P, [(0, 50), (8, 20)], torch.bfloat16, seed=9)
    # (rows between the sequences are not written: start every output at zero)
    a = _run(q, kp, vp, tb, meta, out=torch.zeros_like(q).cuda())
    b = _run(q, kp, vp, tb, meta, out=torch.zeros_like(q).cuda())
    assert torch.equal(a, b)
    from acorninfer_amd.ops.paged_attention import paged_prefill_attention
    qd, kd, vd, td = q.cuda(), kp.cuda(), vp.cuda(), tb.cuda()
    md = [m.cuda() for m in meta]
    out = torch.zeros_like(qd)

    def fn():
        paged_prefill_attention(qd, kd, vd, td, *md, int(meta[2].max()), out=out)

    assert graph_replays_match(fn, lambda: out)
    # a sequence that claims rows past q's end: only rows < R are served
    big = torch.full((q.shape[0] + 16, H, D), 3.0, dtype=q.dtype, device="cuda")
    qv = big[:q.shape[0]]
    qv.copy_(qd)
    outbig = torch.full_like(big, 5.0)
    row0, pos0, nq = meta
    over = (row0.cuda(), pos0.cuda(), (nq + 40).cuda())
    paged_prefill_attention(qv, kd, vd, td, *over, int(nq.max()) + 40, out=outbig[:q.shape[0]])
    torch.cuda.synchronize()
    assert bool((outbig[q.shape[0]:] == 5.0).all())


@pytest.mark.gpu
def test_prefill_attention_contract():
    from acorninfer_amd.ops.paged_attention import paged_prefill_attention, prefill_supported
    assert prefill_supported(torch.bfloat16, 128, 16, 32, 8)
    assert not prefill_supported(torch.float32, 128, 16, 32, 8)
    assert not prefill_supported(torch.bfloat16, 32, 16, 32, 8)
    assert not prefill_supported(torch.bfloat16, 128, 8, 32, 8)
    q, kp, vp, tb, meta = _make(4, 2, 64, 16, [(0, 4)], torch.bfloat16, seed=1)
    with pytest.raises(AssertionError):          # page size not a multiple of 16
        paged_prefill_attention(q.cuda(), kp[:, :8].contiguous().cuda(),
                                vp[:, :8].contiguous().cuda(), tb.cuda(),
                                *[m.cuda() for m in meta], 4)

"""K3 paged decode attention (HIP) vs the oracle restatement of
acorninfer/ops/paged_attention.py:192-216.

CONFIGS are the reference's own (tests/test_ops_paged_attention.py:32-39:
L=1, exactly one page, a one-token tail page, P=4 ragged, empty splits) plus
Qwen3 shapes: GQA 32/8 (rep 4) and 16/8 (rep 2) with D=128, and BASELINE
config 2 at full size (B=8, ctx U[512,4096], 4096-block pool, random
permutation tables). Also: split-count invariance, block relabelling
invariance, determinism, graph replay.
"""
import pytest
import torch

from oracle.ops_ref import paged_attention_ref
from tolerances import TOL_BF16, TOL_F32, max_abs_diff
from gpu_utils import graph_replays_match

# (B, H, KV, D, P, lens, S)
CONFIGS = [
    (1, 4, 2, 16, 16, [1], 1),
    (1, 4, 2, 16, 16, [16], 1),
    (1, 4, 2, 16, 16, [17], 2),
    (2, 4, 2, 16, 4, [7, 20], 2),
    (3, 8, 2, 16, 16, [33, 1, 48], 4),
    (1, 4, 2, 16, 16, [40], 8),
    (2, 32, 8, 128, 16, [1, 300], 1),
    (3, 32, 8, 128, 16, [513, 77, 1024], 8),
    (2, 16, 8, 128, 16, [129, 260], 5),
    (2, 8, 8, 64, 16, [50, 3], 3),
    (2, 64, 8, 128, 16, [100, 31], 2),
    (2, 32, 8, 128, 4, [37, 70], 3),
    (2, 16, 8, 64, 8, [45, 19], 2),
    (1, 8, 1, 128, 32, [95], 1),
]


def _gen(dtype, configs=CONFIGS, seed=23):
    g = torch.Generator().manual_seed(seed)
    for B, H, KV, D, P, lens, S in configs:
        max_pages = max(-(-L // P) for L in lens)
        nb = max_pages + 2
        q = torch.randn(B, H, D, generator=g).to(dtype)
        k_pages = torch.randn(nb, P, KV, D, generator=g).to(dtype)
        v_pages = torch.randn(nb, P, KV, D, generator=g).to(dtype)
        tables = torch.empty(B, max_pages, dtype=torch.int32)
        for i, L in enumerate(lens):
            n = -(-L // P)
            tables[i, :n] = torch.randperm(nb, generator=g)[:n]
            if n < max_pages:
                tables[i, n:] = torch.randint(0, nb, (max_pages - n,), generator=g)
        lens_t = torch.tensor(lens, dtype=torch.int32)
        yield q, k_pages, v_pages, tables, lens_t, S


def _run(q, kp, vp, tb, lens, S):
    from acorninfer_amd.ops.paged_attention import paged_decode_attention
    return paged_decode_attention(q.cuda(), kp.cuda(), vp.cuda(), tb.cuda(), lens.cuda(), S).cpu()


@pytest.mark.gpu
def test_matches_oracle_fp32_tight():
    for args in _gen(torch.float32):
        ref = paged_attention_ref(*args[:5])
        torch.testing.assert_close(_run(*args), ref, **TOL_F32)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_matches_oracle_half(dtype):
    worst = 0.0
    for args in _gen(dtype):
        ref = paged_attention_ref(*args[:5])
        out = _run(*args)
        worst = max(worst, max_abs_diff(out, ref))
        torch.testing.assert_close(out, ref, **TOL_BF16)
    print(f"\n[paged_attn {dtype} max|diff| = {worst:.3g}]")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("direction", [1.0, -1.0])
def test_score_ramps(dtype, direction):
    """Scores that climb (or fall) by ~100 nats along the context: the
    running max moves in many chunks of every wave, so the rescale path is
    exercised throughout, with scores far outside any fixed window."""
    g = torch.Generator().manual_seed(5)
    B, H, KV, D, P, lens = 2, 32, 8, 128, 16, [700, 1000]
    nb = 2 * 63 + 2
    u = torch.ones(D) / D ** 0.5
    q = torch.randn(B, H, D, generator=g) + 2.0 * D ** 0.5 * u
    k_pages = torch.randn(nb, P, KV, D, generator=g)
    v_pages = torch.randn(nb, P, KV, D, generator=g)
    perm = torch.randperm(nb, generator=g)
    tables = torch.zeros(B, 63, dtype=torch.int32)
    off = 0
    for b, L in enumerate(lens):
        n = -(-L // P)
        tables[b, :n] = perm[off:off + n].to(torch.int32)
        for t in range(L):
            ramp = (t / L) if direction > 0 else (1.0 - t / L)
            k_pages[int(tables[b, t // P]), t % P] += 40.0 * ramp * u
        off += n
    args = (q.to(dtype), k_pages.to(dtype), v_pages.to(dtype), tables,
            torch.tensor(lens, dtype=torch.int32))
    ref = paged_attention_ref(*args)
    for S in (1, 3):
        out = _run(*args, S)
        assert torch.isfinite(out).all()
        torch.testing.assert_close(out, ref, **TOL_BF16)


@pytest.mark.gpu
def test_split_count_invariance():
    """The merge is exact up to fp32 rounding: any S gives the same result."""
    q, kp, vp, tb, lens, _ = next(_gen(torch.float32, [(3, 32, 8, 128, 16, [700, 33, 1000], 1)]))
    base = _run(q, kp, vp, tb, lens, 1)
    for S in (2, 3, 7, 16, 63, 64, 100):
        torch.testing.assert_close(_run(q, kp, vp, tb, lens, S), base, **TOL_F32)


@pytest.mark.gpu
def test_block_relabelling_invariance():
    """Permuting the pool's blocks and the table ids together leaves the
    output bitwise unchanged (the kernel reads only through the table)."""
    q, kp, vp, tb, lens, S = next(_gen(torch.bfloat16, [(2, 32, 8, 128, 16, [90, 200], 4)]))
    perm = torch.randperm(kp.shape[0])
    inv = torch.argsort(perm)
    kp2, vp2 = kp[perm], vp[perm]          # block j of kp2 = block perm[j] of kp
    tb2 = inv[tb.long()].to(torch.int32)   # so block b now lives at inv[b]
    assert torch.equal(_run(q, kp, vp, tb, lens, S), _run(q, kp2, vp2, tb2, lens, S))


@pytest.mark.gpu
def test_closed_forms():
    """L=1 -> out = v_0 of the kv head; q=0 -> mean of V over the context."""
    from acorninfer_amd.ops.paged_attention import paged_decode_attention
    g = torch.Generator().manual_seed(1)
    kp = torch.randn(6, 16, 8, 128, generator=g)
    vp = torch.randn(6, 16, 8, 128, generator=g)
    tb = torch.tensor([[4, 1, 0], [2, 5, 3]], dtype=torch.int32)
    q = torch.randn(2, 32, 128, generator=g)
    out = paged_decode_attention(q.cuda(), kp.cuda(), vp.cuda(), tb.cuda(),
                                 torch.tensor([1, 1], dtype=torch.int32).cuda(), 2).cpu()
    for b, blk in enumerate([4, 2]):
        for h in range(32):
            torch.testing.assert_close(out[b, h], vp[blk, 0, h // 4], rtol=0, atol=0)
    out = paged_decode_attention(torch.zeros_like(q).cuda(), kp.cuda(), vp.cuda(), tb.cuda(),
                                 torch.tensor([40, 33], dtype=torch.int32).cuda(), 3).cpu()
    for b, L in enumerate([40, 33]):
        toks = torch.stack([vp[int(tb[b, t // 16]), t % 16] for t in range(L)])  # [L, KV, D]
        mean = toks.double().mean(0)
        for h in range(32):
            torch.testing.assert_close(out[b, h].double(), mean[h // 4], rtol=1e-5, atol=1e-5)


@pytest.mark.gpu
def test_baseline_config2_full_size():
    """B=8, 32/8 heads, D=128, ctx ~U[512,4096], P=16,
    tables = random permutation of a 4096-block pool, K/V ~N(0,1), bf16."""
    from acorninfer_amd.ops.paged_attention import paged_decode_attention, plan_splits
    g = torch.Generator().manual_seed(2024)
    B, H, KV, D, P, NB = 8, 32, 8, 128, 16, 4096
    lens = torch.randint(512, 4097, (B,), generator=g, dtype=torch.int32)
    perm = torch.randperm(NB, generator=g).to(torch.int32)
    tables = torch.zeros(B, NB // B, dtype=torch.int32)
    off = 0
    for b in range(B):
        n = -(-int(lens[b]) // P)
        tables[b, :n] = perm[off:off + n]
        off += n
    kp = torch.randn(NB, P, KV, D, generator=g).bfloat16()
    vp = torch.randn(NB, P, KV, D, generator=g).bfloat16()
    q = torch.randn(B, H, D, generator=g).bfloat16()
    ref = paged_attention_ref(q, kp, vp, tables, lens)
    S = plan_splits(B, KV, int(tables.shape[1]))
    out = paged_decode_attention(q.cuda(), kp.cuda(), vp.cuda(), tables.cuda(), lens.cuda(), S)
    torch.testing.assert_close(out.cpu(), ref, **TOL_BF16)
    rel = ((out.cpu().double() - ref.double()).norm() / ref.double().norm()).item()
    assert rel < 2e-2
    print(f"\n[config2 S={S} max|diff|={max_abs_diff(out, ref):.3g} rel={rel:.3g}]")


@pytest.mark.gpu
@pytest.mark.parametrize("S", [64, 16, 1])
def test_long_context_table_512(S):
    """Configuration 5's contexts: B=8, lengths up to 8192 (one exactly 8192,
    one 8191, one short), tables 512 pages wide over a 4608-block pool. S=64
    is the split cap the decode step uses there (8-page splits, one-wave
    workgroups), S=16 gives 32-page splits (the multi-wave form merged in
    LDS), S=1 one split per sequence over up to 512 pages."""
    from acorninfer_amd.ops.paged_attention import paged_decode_attention, plan_splits
    g = torch.Generator().manual_seed(8192)
    B, H, KV, D, P, W = 8, 32, 8, 128, 16, 512
    lens = torch.randint(1024, 8193, (B,), generator=g, dtype=torch.int32)
    lens[0], lens[1], lens[2] = 8192, 8191, 17
    NB = int(sum(-(-int(n) // P) for n in lens)) + 64
    perm = torch.randperm(NB, generator=g).to(torch.int32)
    tables = torch.randint(0, NB, (B, W), generator=g, dtype=torch.int32)  # junk past the end
    off = 0
    for b in range(B):
        n = -(-int(lens[b]) // P)
        tables[b, :n] = perm[off:off + n]
        off += n
    kp = torch.randn(NB, P, KV, D, generator=g).bfloat16()
    vp = torch.randn(NB, P, KV, D, generator=g).bfloat16()
    q = (torch.randn(B, H, D, generator=g) * 2).bfloat16()
    assert plan_splits(B, KV, W) == 64
    ref = paged_attention_ref(q, kp, vp, tables, lens)
    out = paged_decode_attention(q.cuda(), kp.cuda(), vp.cuda(), tables.cuda(), lens.cuda(), S)
    torch.testing.assert_close(out.cpu(), ref, **TOL_BF16)
    rel = ((out.cpu().double() - ref.double()).norm() / ref.double().norm()).item()
    assert rel < 2e-2
    print(f"\n[ctx<=8192 W=512 S={S} max|diff|={max_abs_diff(out, ref):.3g} rel={rel:.3g}]")


@pytest.mark.gpu
def test_deterministic_and_graph_replay():
    from acorninfer_amd.ops.paged_attention import paged_decode_attention
    q, kp, vp, tb, lens, S = next(_gen(torch.bfloat16, [(3, 32, 8, 128, 16, [513, 77, 1024], 8)]))
    q, kp, vp, tb, lens = (t.cuda() for t in (q, kp, vp, tb, lens))
    a = paged_decode_attention(q, kp, vp, tb, lens, S)
    b = paged_decode_attention(q, kp, vp, tb, lens, S)
    assert torch.equal(a, b)
    out = torch.empty_like(q)
    ws = (torch.empty(3 * 32 * S * 128, device="cuda"), torch.empty(2 * 3 * 32 * S, device="cuda"))
    assert graph_replays_match(
        lambda: paged_decode_attention(q, kp, vp, tb, lens, S, out=out, workspace=ws),
        lambda: out)


def test_num_splits_heuristic_matches_reference_values():
    """The reference's pinned values (tests/test_ops_paged_attention.py:149-154)."""
    from acorninfer_amd.ops.paged_attention import num_splits_for
    assert num_splits_for(1, 8) == 8
    assert num_splits_for(8, 8) == 2
    assert num_splits_for(1, 32) == 4
    assert num_splits_for(4, 32) == 1


def test_build_tables_known_answers():
    """The reference's known answers (tests/test_ops_paged_attention.py:157-191)."""
    from acorninfer_amd.ops.paged_attention import build_tables

    class FakeView:
        def __init__(self, table, L):
            self.table, self._L = table, L

        @property
        def seq_len(self):
            return self._L

    t, lens = build_tables([FakeView([3, 4, 5], 40), FakeView([7], 1)], 16, "cpu")
    assert t.shape == (2, 3) and t.dtype == torch.int32
    assert t[0].tolist() == [3, 4, 5] and t[1].tolist() == [7, 0, 0] and lens.tolist() == [40, 1]

    class _V:
        def __init__(self, table):
            self.table = table

    views = [_V([3, 7, 9]), _V([1])]
    out = torch.full((4, 8), 99, dtype=torch.int32)
    t, lens = build_tables(views, 4, "cpu", lens_override=[11, 2], out=out)
    assert t.data_ptr() == out.data_ptr() and t.shape[0] == 2
    assert out[0, :3].tolist() == [3, 7, 9] and out[0, 3:].tolist() == [0] * 5
    assert out[1, :1].tolist() == [1] and out[1, 1:].tolist() == [0] * 7
    assert out[2:].tolist() == [[99] * 8, [99] * 8]
    assert lens.tolist() == [11, 2] and lens.device.type == "cpu"
    t2, lens2 = build_tables(views, 4, "cpu", lens_override=[11, 2])
    assert t2.tolist() == out[:2, :t2.shape[1]].tolist() and lens2.tolist() == [11, 2]

"""Pins for oracle/ops_ref.py (CPU). Each check is chosen so that a plausible
restatement mistake (dropped term, wrong sign/index, transposed operand)
fails it: float64 closed forms, the reference's known answers, brute force."""
import math

import torch

from oracle.ops_ref import (build_tables_ref, fused_add_rmsnorm_ref, inv_freq_ref,
                            num_splits_ref, paged_attention_brute, paged_attention_ref,
                            qknorm_rope_ref, rmsnorm_ref, rope_ref)


def test_rmsnorm_float64_closed_form():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(3, 100, generator=g)
    w = torch.randn(100, generator=g)
    ref = x.double() / (x.double().pow(2).mean(-1, keepdim=True) + 1e-6).sqrt() * w.double()
    torch.testing.assert_close(rmsnorm_ref(x, w, 1e-6).double(), ref, rtol=1e-6, atol=1e-6)
    n, r = fused_add_rmsnorm_ref(x, None, w, 1e-6)
    assert torch.equal(r, x)
    torch.testing.assert_close(n, rmsnorm_ref(x, w, 1e-6))
    # with a residual: normalises the SUM (a dropped residual term fails here)
    res = torch.randn(3, 100, generator=g)
    n2, r2 = fused_add_rmsnorm_ref(x, res, w, 1e-6)
    torch.testing.assert_close(r2, x + res)
    torch.testing.assert_close(n2, rmsnorm_ref(x + res, w, 1e-6))
    # scale invariance (eps small relative to mean square)
    torch.testing.assert_close(rmsnorm_ref(4 * x, w, 0.0), rmsnorm_ref(x, w, 0.0))


def test_rmsnorm_bf16_rounds_once_at_the_end():
    x = torch.tensor([[1.0, 2.0, 3.0, 4.0]]).bfloat16()
    w = torch.ones(4).bfloat16()
    expect = (x.float() / math.sqrt((1 + 4 + 9 + 16) / 4 + 1e-6)).bfloat16()
    assert torch.equal(rmsnorm_ref(x, w, 1e-6), expect)


def test_rope_known_answer_first_pair_rotates_by_position():
    """The reference's test_qwen3_model.py:64-82: inv_freq[0] == 1, so the
    (x[0], x[D/2]) pair rotates by exactly `pos` radians."""
    D = 16
    inv = inv_freq_ref(D, 1e6)
    assert inv[0] == 1.0
    assert torch.allclose(inv[1], torch.tensor(1e6 ** (-2 / D)))
    x = torch.zeros(1, 1, 1, D)
    x[0, 0, 0, 0] = 1.0
    for pos in (0, 1, 5, 100):
        y = rope_ref(x, torch.tensor([pos]), inv)
        assert abs(float(y[0, 0, 0, 0]) - math.cos(pos)) < 1e-6
        assert abs(float(y[0, 0, 0, D // 2]) - math.sin(pos)) < 1e-6


def test_rope_float64_rotation_and_norm():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(2, 3, 1, 32, generator=g)
    pos = torch.tensor([7, 1234])
    inv = inv_freq_ref(32, 1e4)
    y = rope_ref(x, pos, inv).double()
    ang = pos.double()[:, None] * inv.double()[None, :]            # [B, D/2]
    c, s = ang.cos()[:, None, None, :], ang.sin()[:, None, None, :]
    x1, x2 = x.double()[..., :16], x.double()[..., 16:]
    ref = torch.cat((x1 * c - x2 * s, x2 * c + x1 * s), dim=-1)
    torch.testing.assert_close(y, ref, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(y.norm(dim=-1), x.double().norm(dim=-1), rtol=1e-5, atol=1e-5)
    assert torch.equal(rope_ref(x, torch.zeros(2, dtype=torch.long), inv), x)


def test_rope_bf16_three_step_rounding():
    x = torch.tensor([[[[1.5, -0.75, 2.25, 0.3]]]]).bfloat16()
    pos = torch.tensor([3])
    inv = inv_freq_ref(4, 10.0)
    ang = (pos.float()[:, None] * inv[None, :])
    c = torch.cat((ang, ang), -1).cos().bfloat16().float()
    s = torch.cat((ang, ang), -1).sin().bfloat16().float()
    xf = x.float()[0, 0, 0]
    rot = torch.cat((-xf[2:], xf[:2]))
    expect = ((xf * c[0]).bfloat16().float() + (rot * s[0]).bfloat16().float()).bfloat16()
    assert torch.equal(rope_ref(x, pos, inv)[0, 0, 0], expect)


def test_qknorm_rope_is_norm_then_rope():
    g = torch.Generator().manual_seed(2)
    q = torch.randn(2, 4, 1, 16, generator=g)
    k = torch.randn(2, 2, 1, 16, generator=g)
    qw, kw = torch.randn(16, generator=g), torch.randn(16, generator=g)
    pos, inv = torch.tensor([3, 9]), inv_freq_ref(16, 1e6)
    qo, ko = qknorm_rope_ref(q, k, qw, kw, 1e-6, pos, inv)
    torch.testing.assert_close(qo, rope_ref(rmsnorm_ref(q, qw, 1e-6), pos, inv))
    torch.testing.assert_close(ko, rope_ref(rmsnorm_ref(k, kw, 1e-6), pos, inv))


def _attn_case(seed, B, H, KV, D, P, lens):
    g = torch.Generator().manual_seed(seed)
    maxp = max(-(-L // P) for L in lens)
    nb = maxp * B + 1
    q = torch.randn(B, H, D, generator=g)
    kp = torch.randn(nb, P, KV, D, generator=g)
    vp = torch.randn(nb, P, KV, D, generator=g)
    perm = torch.randperm(nb, generator=g)
    tb = torch.zeros(B, maxp, dtype=torch.int32)
    for b in range(B):
        n = -(-lens[b] // P)
        tb[b, :n] = perm[b * maxp: b * maxp + n]
    return q, kp, vp, tb, torch.tensor(lens, dtype=torch.int32)


def test_paged_attention_ref_vs_brute_force():
    for args in (_attn_case(0, 2, 4, 2, 16, 4, [7, 13]), _attn_case(1, 1, 8, 2, 8, 16, [33]),
                 _attn_case(2, 3, 6, 3, 4, 2, [1, 5, 9])):
        torch.testing.assert_close(paged_attention_ref(*args).double(),
                                   paged_attention_brute(*args), rtol=1e-5, atol=1e-5)


def test_paged_attention_ref_closed_forms():
    q, kp, vp, tb, _ = _attn_case(3, 2, 4, 2, 16, 4, [9, 9])
    out = paged_attention_ref(q, kp, vp, tb, torch.tensor([1, 1], dtype=torch.int32))
    for b in range(2):
        for h in range(4):  # GQA: head h reads kv h // 2
            assert torch.equal(out[b, h], vp[int(tb[b, 0]), 0, h // 2])
    out = paged_attention_ref(torch.zeros_like(q), kp, vp, tb, torch.tensor([9, 5], dtype=torch.int32))
    for b, L in enumerate([9, 5]):
        toks = torch.stack([vp[int(tb[b, t // 4]), t % 4] for t in range(L)])
        for h in range(4):
            torch.testing.assert_close(out[b, h], toks[:, h // 2].mean(0), rtol=1e-6, atol=1e-6)


def test_num_splits_and_build_tables_known_answers():
    assert [num_splits_ref(1, 8), num_splits_ref(8, 8), num_splits_ref(1, 32),
            num_splits_ref(4, 32)] == [8, 2, 4, 1]
    t, lens = build_tables_ref([[3, 4, 5], [7]], [40, 1], 16)
    assert t.tolist() == [[3, 4, 5], [7, 0, 0]] and lens.tolist() == [40, 1]

"""K3 running the qkv epilogue itself (acorn_paged_attention_qkv) against
the two launches it replaces in the decode step (acorn_qkv_epilogue, then
acorn_paged_attention): the same output bits and the same pool bits. The
fused output is also checked against the oracle directly: q/k/v from the
split-ordered sum of the partials (qwen3.py:180-192), oracle.ops_ref's
q/k RMSNorm + RoPE, the new k/v written at (page, slot) (pager.py:87-113),
then oracle.ops_ref.paged_attention_ref (paged_attention.py:192-216).
All calls go through the C-ABI."""
import pytest
import torch

from acorninfer_amd import _lib
from oracle.ops_ref import inv_freq_ref, paged_attention_ref, qknorm_rope_ref
from tolerances import TOL_BF16


def test_supported_predicate():
    f = _lib.lib().acorn_paged_attention_qkv_supported
    BF, F16, F32 = _lib.BF16, _lib.F16, _lib.F32
    assert f(32, 8, 128, 16, 48, 12, BF, BF) == 1
    assert f(32, 8, 128, 16, 48, 12, F16, F16) == 1
    assert f(32, 8, 64, 32, 48, 3, BF, BF) == 1        # 16-page splits of 32-token pages
    assert f(32, 8, 128, 16, 48, 12, F32, F32) == 0     # fp32 has no MFMA K3
    assert f(32, 8, 128, 16, 48, 12, BF, F32) == 0      # norm weights of another dtype
    assert f(32, 8, 128, 8, 48, 12, BF, BF) == 0        # pages of 8 tokens
    assert f(32, 8, 128, 16, 256, 8, BF, BF) == 1       # 32-page splits: 8-wave workgroups
    assert f(32, 8, 128, 16, 640, 1, BF, BF) == 1       # one split of 640 pages
    assert f(32, 8, 128, 16, 30000, 1, BF, BF) == 0     # block ids past the LDS budget
    assert f(32, 8, 256, 16, 48, 12, BF, BF) == 0
    assert f(48, 8, 128, 16, 48, 12, BF, BF) == 0       # 6 q heads per kv head


# (B, H, KV, D, P, lens, table_stride, S, ksplit of the qkv partials)
CASES = [
    (3, 8, 2, 128, 16, [1, 16, 17], 8, 2, 1),            # first token, page end, page start
    (2, 32, 8, 128, 16, [100, 128], 8, 8, 4),            # one-page splits, full table
    (4, 16, 8, 128, 16, [33, 64, 65, 2], 6, 3, 6),       # ksplit 6: past the first batch
    (2, 8, 8, 64, 16, [31, 48], 4, 1, 3),                # D 64, one kv head per q head
    (2, 16, 2, 128, 32, [40, 95], 4, 2, 2),              # 32-token pages, 8 q heads per kv
    # 8-wave workgroups (splits of more than 16 pages): the new token's wave
    # writes it; waves past the sequence's pages only join the LDS merge
    (2, 32, 8, 128, 16, [300, 513], 40, 1, 2),           # one split, owners waves 3 and 6
    (3, 16, 8, 128, 16, [1, 64, 200], 20, 1, 1),         # a one-token sequence: wave 0
    (2, 32, 8, 128, 16, [700, 1000], 80, 2, 3),          # 40-page splits, combine after
    (2, 32, 8, 128, 16, [5000, 9000], 1100, 1, 2),       # 138 pages a wave: ids staged in LDS
    # head groups (one split over <= 64 pages, few (sequence, kv head) pairs): each kv
    # head's q heads in G workgroups of their own
    (1, 32, 4, 128, 16, [70], 6, 1, 2),                  # G = 8, one q head each, one wave
    (1, 32, 4, 128, 16, [300], 20, 1, 2),                # G = 8, eight-wave workgroups
    (2, 16, 4, 64, 32, [100, 300], 12, 1, 1),            # D 64, 32-token pages, G = 4
]


def _case(dtype, B, H, KV, D, P, lens, ts, ks, seed):
    g = torch.Generator().manual_seed(seed)
    nb = B * ts + 3
    width = (H + 2 * KV) * D
    part = torch.randn(ks, B, width, generator=g) * 0.5
    q_w = (1.0 + 0.2 * torch.randn(D, generator=g)).to(dtype)
    k_w = (1.0 + 0.2 * torch.randn(D, generator=g)).to(dtype)
    kp = torch.randn(nb, P, KV, D, generator=g).to(dtype)
    vp = torch.randn(nb, P, KV, D, generator=g).to(dtype)
    perm = torch.randperm(nb, generator=g)
    tables = perm[:B * ts].view(B, ts).to(torch.int32).contiguous()
    lens_t = torch.tensor(lens, dtype=torch.int32)
    pos = (lens_t - 1).to(torch.int64)
    pages = torch.tensor([int(tables[b, (L - 1) // P]) for b, L in enumerate(lens)],
                         dtype=torch.int64)
    slots = torch.tensor([(L - 1) % P for L in lens], dtype=torch.int64)
    inv_freq = inv_freq_ref(D, 1e6).float()
    return part, q_w, k_w, kp, vp, tables, lens_t, pos, pages, slots, inv_freq, nb


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("case", CASES)
def test_fused_matches_two_launches_and_oracle(dtype, case):
    B, H, KV, D, P, lens, ts, S, ks = case
    eps = 1e-6
    part, q_w, k_w, kp, vp, tables, lens_t, pos, pages, slots, inv_freq, nb = _case(
        dtype, B, H, KV, D, P, lens, ts, ks, seed=sum(lens) + ks)
    L = _lib.lib()
    ptr, dt = _lib.ptr, _lib.dtype_code(kp)
    dev = torch.device("cuda:0")
    part_d, qw_d, kw_d = part.to(dev), q_w.to(dev), k_w.to(dev)
    tb_d, ln_d, pos_d = tables.to(dev), lens_t.to(dev), pos.to(dev)
    pg_d, sl_d, fr_d = pages.to(dev), slots.to(dev), inv_freq.to(dev)
    st = _lib.stream_ptr(dev)
    print(f"case {case} {dtype}", flush=True)

    # the two launches of the unfused step
    kpa, vpa = kp.to(dev), vp.to(dev)
    q = torch.empty(B, H, D, dtype=dtype, device=dev)
    out_a = torch.empty(B, H, D, dtype=dtype, device=dev)
    ws_a = torch.empty(B * H * S * D, device=dev)
    ml_a = torch.empty(2 * B * H * S, device=dev)
    _lib.check(L.acorn_qkv_epilogue(ptr(part_d), ks, ptr(q), ptr(kpa), ptr(vpa), ptr(pg_d),
                                    ptr(sl_d), B, H, KV, D, P, nb, ptr(qw_d), ptr(kw_d), eps,
                                    ptr(pos_d), ptr(fr_d), dt, dt, st), "qkv_epilogue")
    _lib.check(L.acorn_paged_attention(ptr(q), ptr(kpa), ptr(vpa), ptr(tb_d), ptr(ln_d),
                                       ptr(out_a), ptr(ws_a), ptr(ml_a), B, H, KV, D, P, nb, ts,
                                       S, D ** -0.5, dt, st), "K3")
    # the fused launch
    kpb, vpb = kp.to(dev), vp.to(dev)
    out_b = torch.empty(B, H, D, dtype=dtype, device=dev)
    ws_b = torch.empty(B * H * S * D, device=dev)
    ml_b = torch.empty(2 * B * H * S, device=dev)
    _lib.check(L.acorn_paged_attention_qkv(
        ptr(part_d), ks, ptr(kpb), ptr(vpb), ptr(pg_d), ptr(sl_d), ptr(tb_d), ptr(ln_d),
        ptr(out_b), ptr(ws_b), ptr(ml_b), B, H, KV, D, P, nb, ts, S, D ** -0.5, ptr(qw_d),
        ptr(kw_d), eps, ptr(pos_d), ptr(fr_d), dt, dt, st), "K3+epilogue")
    torch.cuda.synchronize()
    assert torch.equal(out_a.view(torch.int16), out_b.view(torch.int16))
    assert torch.equal(kpa.view(torch.int16), kpb.view(torch.int16))
    assert torch.equal(vpa.view(torch.int16), vpb.view(torch.int16))

    # oracle: split-ordered sum, rounded; norm + RoPE; scatter; attention
    acc = part[0].clone()
    for s in range(1, ks):
        acc = acc + part[s]
    x = acc.to(dtype).view(B, H + 2 * KV, D)
    qn, kn = qknorm_rope_ref(x[:, :H, None, :], x[:, H:H + KV, None, :], q_w, k_w, eps, pos,
                             inv_freq)
    kp_ref, vp_ref = kp.clone(), vp.clone()
    for b in range(B):
        kp_ref[pages[b], slots[b]] = kn[b, :, 0]
        vp_ref[pages[b], slots[b]] = x[b, H + KV:]
    ref = paged_attention_ref(qn[:, :, 0], kp_ref, vp_ref, tables, lens_t)
    assert torch.allclose(out_b.cpu().float(), ref.float(), **TOL_BF16)
    assert torch.allclose(kpb.cpu().float(), kp_ref.float(), **TOL_BF16)
    assert torch.equal(vpb.cpu().view(torch.int16), vp_ref.view(torch.int16))


def test_fused_rejects_unsupported_without_launching():
    # pages of 8 tokens: refused before any pointer is read or any launch
    L = _lib.lib()
    rc = L.acorn_paged_attention_qkv(None, 1, None, None, None, None, None, None, None, None,
                                     None, 2, 32, 8, 128, 8, 16, 8, 2, 0.1, None, None, 1e-6,
                                     None, None, _lib.BF16, _lib.BF16, None)
    with pytest.raises(NotImplementedError):
        _lib.check(rc, "K3+epilogue")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_qkv_epilogue_row_form_equals_per_head_form(dtype):
    """At prefill sizes (256+ rows, one split, head_dim 128) the qkv epilogue
    runs one wave per token row (cos/sin once per row); below, one wave per
    (row, head). 300 rows in one call against the same rows as two calls of
    150: the same q bits and pool bits, and q against the oracle's norm + RoPE
    (positions up to 8191, where the angles are largest). Rows 7 and 200 carry
    a page outside the pool: nothing is written for them."""
    B, H, KV, D, P = 300, 32, 8, 128, 16
    eps = 1e-6
    g = torch.Generator().manual_seed(91)
    nb = B // P + 4
    width = (H + 2 * KV) * D
    part = torch.randn(1, B, width, generator=g) * 0.5
    q_w = (1.0 + 0.2 * torch.randn(D, generator=g)).to(dtype)
    k_w = (1.0 + 0.2 * torch.randn(D, generator=g)).to(dtype)
    pos = torch.randint(0, 8192, (B,), generator=g, dtype=torch.int64)
    pages = torch.randperm(nb, generator=g)[:B // P + 1].repeat_interleave(P)[:B].clone()
    slots = torch.arange(B, dtype=torch.int64) % P
    pages[7] = nb + 5
    pages[200] = -1
    inv_freq = inv_freq_ref(D, 1e6).float()
    L = _lib.lib()
    ptr, dt = _lib.ptr, _lib.dtype_code(torch.empty(0, dtype=dtype))
    dev = torch.device("cuda:0")
    st = _lib.stream_ptr(dev)
    part_d, qw_d, kw_d = part.to(dev), q_w.to(dev), k_w.to(dev)
    pos_d, pg_d, sl_d, fr_d = pos.to(dev), pages.to(dev), slots.to(dev), inv_freq.to(dev)
    pools = []
    outs = []
    for chunks in ((0, B), (0, 150, B)):
        kp = torch.full((nb, P, KV, D), 7.0, dtype=dtype, device=dev)
        vp = torch.full((nb, P, KV, D), 7.0, dtype=dtype, device=dev)
        q = torch.empty(B, H, D, dtype=dtype, device=dev)
        for a, b in zip(chunks[:-1], chunks[1:]):
            n = b - a
            _lib.check(L.acorn_qkv_epilogue(
                ptr(part_d[:, a:b].contiguous()), 1, ptr(q[a:b]), ptr(kp), ptr(vp),
                ptr(pg_d[a:b]), ptr(sl_d[a:b]), n, H, KV, D, P, nb, ptr(qw_d), ptr(kw_d), eps,
                ptr(pos_d[a:b]), ptr(fr_d), dt, dt, st), "qkv_epilogue")
        torch.cuda.synchronize()
        outs.append(q.cpu())
        pools.append((kp.cpu(), vp.cpu()))
    iv = torch.int16 if dtype != torch.float32 else torch.int32
    assert torch.equal(outs[0].view(iv), outs[1].view(iv))
    for a, b in zip(pools[0], pools[1]):
        assert torch.equal(a.view(iv), b.view(iv))
    x = part[0].to(dtype).view(B, H + 2 * KV, D)
    qn, _ = qknorm_rope_ref(x[:, :H, None, :], x[:, H:H + KV, None, :], q_w, k_w, eps, pos,
                            inv_freq)
    tol = TOL_BF16 if dtype != torch.float32 else dict(rtol=1e-5, atol=1e-5)
    assert torch.allclose(outs[0].float(), qn[:, :, 0].float(), **tol)
    # the rows with a page outside the pool wrote nothing; the others did
    kp0 = pools[0][0]
    assert bool((kp0 == 7.0).sum() == (nb * P - (B - 2)) * KV * D)

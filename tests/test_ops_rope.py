"""K2 RoPE and fused qk-norm + RoPE (HIP) vs the oracle restatements of
acorninfer/ops/rope.py:116-125 and models/qwen3.py:50-60 (cases as the
reference's tests/test_ops_rope.py:9 plus Qwen3-8B heads, theta 1e6)."""
import pytest
import torch

from oracle.ops_ref import inv_freq_ref, qknorm_rope_ref, rope_ref
from tolerances import MAX_ONE_ULP_FRACTION, TOL_BF16, TOL_F32, max_abs_diff, ulp_distance

CASES = [(1, 4, 16, 1e4), (2, 4, 16, 1e4), (3, 8, 16, 1e4), (4, 32, 128, 1e4),
         (8, 32, 128, 1e6), (8, 8, 128, 1e6)]


def _gen(dtype):
    g = torch.Generator().manual_seed(11)
    for B, H, D, theta in CASES:
        x = torch.randn(B, H, 1, D, generator=g).to(dtype)
        pos = torch.arange(B) * 3 + 5                      # non-zero start
        if theta == 1e6:
            pos = torch.randint(512, 8192, (B,), generator=g)  # long-context positions
        yield x, pos, inv_freq_ref(D, theta)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_rope_matches_oracle(dtype):
    from acorninfer_amd.ops.rope import fused_rope_inplace
    worst, mism, total = 0.0, 0, 0
    for x, pos, inv in _gen(dtype):
        ref = rope_ref(x, pos, inv)
        q = x.clone().cuda()
        k = x.clone().cuda()
        fused_rope_inplace(q, k, pos.cuda(), inv.cuda())
        tol = TOL_F32 if dtype == torch.float32 else TOL_BF16
        torch.testing.assert_close(q.cpu(), ref, **tol)
        assert torch.equal(q, k)
        worst = max(worst, max_abs_diff(q, ref))
        mism += int((q.cpu() != ref).sum())
        total += ref.numel()
    print(f"\n[rope {dtype} max|diff| = {worst:.3g}; {mism}/{total} elements differ]")
    if dtype != torch.float32:
        # the reference's bitwise target (tests/test_ops_rope.py:32-55): the
        # same three roundings of the same fp32 values, so the same bits
        assert mism == 0, f"{mism}/{total} elements differ"


@pytest.mark.gpu
def test_rope_int32_positions_and_position_zero_identity():
    from acorninfer_amd.ops.rope import fused_rope_inplace
    x = torch.randn(2, 4, 1, 128).bfloat16()
    q = x.clone().cuda()
    k = x[:, :2].clone().cuda()
    fused_rope_inplace(q, k, torch.zeros(2, dtype=torch.int32, device="cuda"),
                       inv_freq_ref(128, 1e6).cuda())
    assert torch.equal(q.cpu(), x)  # cos(0)=1, sin(0)=0 exactly
    assert torch.equal(k.cpu(), x[:, :2])


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_qknorm_rope_matches_oracle(dtype):
    from acorninfer_amd.ops.rope import qknorm_rope_inplace
    g = torch.Generator().manual_seed(13)
    for B, H, KV, D in [(1, 4, 2, 16), (8, 32, 8, 128), (3, 16, 8, 128)]:
        q = torch.randn(B, H, 1, D, generator=g).to(dtype)
        k = torch.randn(B, KV, 1, D, generator=g).to(dtype)
        qw = (1 + 0.1 * torch.randn(D, generator=g)).to(dtype)
        kw = (1 + 0.1 * torch.randn(D, generator=g)).to(dtype)
        pos = torch.randint(0, 4096, (B,), generator=g)
        inv = inv_freq_ref(D, 1e6)
        q_ref, k_ref = qknorm_rope_ref(q, k, qw, kw, 1e-6, pos, inv)
        qd, kd = q.cuda(), k.cuda()
        qknorm_rope_inplace(qd, kd, qw.cuda(), kw.cuda(), 1e-6, pos.cuda(), inv.cuda())
        tol = TOL_F32 if dtype == torch.float32 else TOL_BF16
        torch.testing.assert_close(qd.cpu(), q_ref, **tol)
        torch.testing.assert_close(kd.cpu(), k_ref, **tol)
        if dtype == torch.bfloat16:
            for got, want in ((qd, q_ref), (kd, k_ref)):
                d = ulp_distance(got, want)
                print(f"\n[qknorm+rope bf16 B={B} H={H}: {int((d > 0).sum())}/{d.numel()} "
                      f"elements differ, max {int(d.max())} ulp]")
                # the norm may land one ulp off (reduction order, rsqrt);
                # RoPE's two rounded products can carry that to two
                assert int(d.max()) <= 2
                assert int((d > 0).sum()) <= MAX_ONE_ULP_FRACTION * d.numel() + 1


@pytest.mark.gpu
def test_rope_contract_asserts():
    from acorninfer_amd.ops.rope import fused_rope_inplace
    q = torch.randn(2, 4, 2, 16, device="cuda")  # s == 2
    with pytest.raises(AssertionError):
        fused_rope_inplace(q, q, torch.zeros(2, device="cuda"), inv_freq_ref(16, 1e4))

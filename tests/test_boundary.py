"""The rest of the drop-in boundary: the exported torch `_ref` functions,
the bf16 decode-GEMM module (acorninfer/ops/decode_gemm.py: triton_gemm,
linear_dispatch, configure) and the model hook dispatch_linear
(acorninfer/models/qwen3.py:21-47).

- the `_ref` functions are checked against the oracle restatements (bitwise
  for K1/K2, whose formulas fix every rounding; fp32 tolerance for K3);
- linear_dispatch with layout "none" is F.linear byte for byte (the
  reference's hard gate, tests/test_decode_gemm.py);
- the kernel path is checked against the fp32 matmul of the same bf16
  operands with the reference's TOL_BF16_GEMM (rtol 2e-2, atol 1e-2,
  tests/test_decode_gemm.py:53-61) and the north-star 1e-2 norm-wise bar;
- dispatch_linear: unmarked modules run their own forward; w8a16 / w4a16
  markers route to the quant GEMMs (within the GEMM bar of the dequantised
  weight); unknown markers and shapes raise ValueError.
"""
import pytest
import torch

from oracle.ops_ref import fused_add_rmsnorm_ref as k1_oracle
from oracle.ops_ref import inv_freq_ref, paged_attention_ref, rope_ref
from tolerances import GEMM_REL, TOL_F32, rel_err
from gpu_utils import graph_replays_match

TOL_BF16_GEMM = dict(rtol=2e-2, atol=1e-2)


# ------------------------------------------------------------ CPU ---------

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("with_res", [False, True])
def test_rmsnorm_ref_export_equals_oracle(dtype, with_res):
    from acorninfer_amd.ops.rmsnorm import fused_add_rmsnorm_ref
    g = torch.Generator().manual_seed(3)
    x = torch.randn(5, 256, generator=g).to(dtype)
    r = torch.randn(5, 256, generator=g).to(dtype) if with_res else None
    w = torch.randn(256, generator=g).to(dtype)
    a = fused_add_rmsnorm_ref(x, r, w, 1e-6)
    b = k1_oracle(x, r, w, 1e-6)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rope_ref_export_equals_oracle(dtype):
    from acorninfer_amd.ops.rope import fused_rope_ref
    g = torch.Generator().manual_seed(4)
    x = torch.randn(3, 8, 1, 128, generator=g).to(dtype)
    pos = torch.tensor([0, 17, 4095])
    inv = inv_freq_ref(128, 1e6)
    assert torch.equal(fused_rope_ref(x, pos, inv), rope_ref(x, pos, inv))


def test_attention_ref_export_matches_oracle():
    from acorninfer_amd.ops.paged_attention import paged_decode_attention_ref
    g = torch.Generator().manual_seed(5)
    B, H, KV, D, P = 3, 8, 2, 64, 4
    lens = torch.tensor([1, 9, 16], dtype=torch.int32)
    kp = torch.randn(12, P, KV, D, generator=g)
    vp = torch.randn(12, P, KV, D, generator=g)
    q = torch.randn(B, H, D, generator=g)
    tables = torch.stack([torch.randperm(12, generator=g)[:4] for _ in range(B)]).to(torch.int32)
    torch.testing.assert_close(paged_decode_attention_ref(q, kp, vp, tables, lens),
                               paged_attention_ref(q, kp, vp, tables, lens), **TOL_F32)


def test_linear_dispatch_none_is_f_linear_bytewise():
    from acorninfer_amd.ops import decode_gemm as dg
    dg.reset()
    g = torch.Generator().manual_seed(6)
    x = torch.randn(2, 3, 64, generator=g).bfloat16()
    w = torch.randn(32, 64, generator=g).bfloat16()
    assert torch.equal(dg.linear_dispatch(x, w, "qo"), torch.nn.functional.linear(x, w))
    assert dg.configure("none", {"qo": (32, 64)}) == {"layout": "none"}
    assert torch.equal(dg.linear_dispatch(x, w, "qo"), torch.nn.functional.linear(x, w))


def test_dispatch_linear_markers_cpu():
    from acorninfer_amd.models.qwen3 import dispatch_linear
    g = torch.Generator().manual_seed(7)
    lin = torch.nn.Linear(64, 32, bias=False)
    x = torch.randn(4, 64, generator=g)
    assert torch.equal(dispatch_linear(lin, x), lin(x))        # unmarked: own forward
    lin._m7_quant = "int3"
    with pytest.raises(ValueError):
        dispatch_linear(lin, x)
    lin._m7_quant = "w8a16"                                    # (32, 64) is not a class
    with pytest.raises(ValueError):
        dispatch_linear(lin, x)


# ------------------------------------------------------------ GPU ---------

SHAPES = {"qo": (4096, 4096), "kv": (1024, 4096), "gate_up": (12288, 4096),
          "down": (4096, 12288)}


@pytest.mark.gpu
@pytest.mark.parametrize("cls", list(SHAPES))
def test_triton_gemm_matches_fp32(cls):
    from acorninfer_amd.ops import decode_gemm as dg
    dg.reset()
    N, K = SHAPES[cls]
    g = torch.Generator().manual_seed(11)
    w = torch.randn(N, K, generator=g).bfloat16()
    wd = w.cuda()
    for M in (1, 2, 4, 8, 16):
        x = torch.randn(M, K, generator=g).bfloat16()
        ref = x.float() @ w.float().T
        out = dg.triton_gemm(x.cuda(), wd, cls).float().cpu()
        torch.testing.assert_close(out, ref, **TOL_BF16_GEMM)
        assert rel_err(out, ref) <= GEMM_REL
    # an explicit reference-style cfg: only SPLIT_K carries over
    x = torch.randn(3, K, generator=g).bfloat16()
    out = dg.triton_gemm(x.cuda(), wd, cls, cfg=(64, 64, 4, 3, 2)).float().cpu()
    torch.testing.assert_close(out, x.float() @ w.float().T, **TOL_BF16_GEMM)


@pytest.mark.gpu
def test_triton_gemm_graph_replay():
    from acorninfer_amd.ops import decode_gemm as dg
    dg.reset()
    w = torch.randn(4096, 12288, device="cuda").bfloat16()
    x = torch.randn(8, 12288, device="cuda").bfloat16()
    out = torch.empty(8, 4096, device="cuda", dtype=torch.bfloat16)
    assert graph_replays_match(lambda: dg.triton_gemm(x, w, "down", out=out), lambda: out)


@pytest.mark.gpu
def test_configure_table_and_dispatch():
    from acorninfer_amd.ops import decode_gemm as dg
    rep = dg.configure("triton", {"qo": (4096, 4096)}, buckets=(1, 8), verbose=False)
    row = rep["classes"]["qo"]["rows"][8]
    assert {"triton_us", "tn_us", "best_cublas_us", "win_vs_best_pct", "adopted_m",
            "table"} <= set(row)
    w = torch.randn(4096, 4096, device="cuda").bfloat16()
    for M in (1, 8):
        x = torch.randn(M, 4096, device="cuda").bfloat16()
        got = dg.linear_dispatch(x, w, "qo")
        if "qo" in dg._state["active"] and dg._state["table"][("qo", M)] == "triton":
            assert torch.equal(got, dg.triton_gemm(x, w, "qo"))
        else:
            assert torch.equal(got, torch.nn.functional.linear(x, w))
    # forcing the table: the kernel path runs and matches the fp32 product
    dg._state["active"].add("qo")
    dg._state["table"][("qo", 8)] = "triton"
    x = torch.randn(2, 4, 4096, device="cuda").bfloat16()         # M = 8 through a 3-D view
    got = dg.linear_dispatch(x, w, "qo")
    assert got.shape == (2, 4, 4096)
    assert torch.equal(got.view(8, 4096), dg.triton_gemm(x.view(8, 4096), w, "qo"))
    dg.reset()


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["w8a16", "w4a16"])
def test_dispatch_linear_quantised(mode):
    from acorninfer_amd.models.qwen3 import dispatch_linear
    from acorninfer_amd.quant.quantize import apply_quant
    from oracle.quant_ref import dequant_w4_sym_ref, dequant_w8_ref, unpack_w4_ref

    class Attn(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.q_proj = torch.nn.Linear(4096, 4096, bias=False)

    torch.manual_seed(0)
    m = Attn()
    with torch.no_grad():
        m.q_proj.weight.normal_(0, 0.02)
    m = m.to(torch.bfloat16)
    apply_quant(m, mode)
    lin = m.q_proj
    if mode == "w8a16":
        wd = torch.from_numpy(dequant_w8_ref(lin.weight.data.numpy(), lin._q_scale.numpy())).float()
    else:
        u = unpack_w4_ref(lin.weight.data.numpy())
        wd = torch.from_numpy(dequant_w4_sym_ref(u, lin._q_scale.numpy())).float()
    lin.weight.data = lin.weight.data.cuda()
    lin._q_scale = lin._q_scale.cuda()
    x = torch.randn(2, 3, 4096).bfloat16()
    out = dispatch_linear(lin, x.cuda())
    assert out.shape == (2, 3, 4096) and out.dtype == torch.bfloat16
    ref = x.float().view(6, 4096) @ wd.T
    assert rel_err(out.float().cpu().view(6, 4096), ref) <= GEMM_REL

"""The quantised safetensors format (models/checkpoint.py), on the CPU: a
model written by save_quantized and read back by load_quantized holds the
same bytes in every weight, scale and norm, in the same fused and
interleaved layout, for bf16, w8a16 and w4a16; the file keeps the
reference's module names and the int4 packing of quant/quantize.py:85-101
(unpacking a stored q_proj gives the quantiser's own nibbles)."""
import pytest
import torch

from acorninfer_amd.config import Qwen3Config
from acorninfer_amd.models.checkpoint import load_quantized, save_quantized
from acorninfer_amd.models.qwen3 import Qwen3DecodeModel, random_state_dict
from acorninfer_amd.quant import quantize as Q


def _model(fmt):
    cfg = Qwen3Config.qwen3_0_6b().with_layers(2)
    sd = random_state_dict(cfg, seed=4, std=0.02, dtype=torch.float32)
    return cfg, sd, Qwen3DecodeModel.from_state_dict(cfg, sd, weight_format=fmt, device="cpu")


def _same(a, b):
    assert (a is None) == (b is None)
    if a is not None:
        assert a.dtype == b.dtype and a.shape == b.shape and torch.equal(a, b)


@pytest.mark.parametrize("fmt", ["bf16", "w8a16", "w4a16"])
def test_round_trip_is_bit_exact(fmt, tmp_path):
    cfg, _, m = _model(fmt)
    path = str(tmp_path / "model.safetensors")
    save_quantized(m, path)
    r = load_quantized(path, device="cpu")
    assert r.cfg == cfg
    _same(r.embed, m.embed)
    _same(r.norm, m.norm)
    for La, Lb in zip(m.layers, r.layers):
        for n in ("input_norm", "post_norm", "q_norm", "k_norm"):
            _same(getattr(Lb, n), getattr(La, n))
        for n in ("qkv", "o", "gate_up", "down"):
            a, b = getattr(La, n), getattr(Lb, n)
            assert (a.fmt, a.N, a.K, a.il16) == (b.fmt, b.N, b.K, b.il16)
            _same(b.w, a.w)
            _same(b.scale, a.scale)
            _same(b.zero, a.zero)
    _same(r.lm_head.w, m.lm_head.w)
    _same(r.lm_head.scale, m.lm_head.scale)


def test_file_uses_reference_names_and_packing(tmp_path):
    from safetensors import safe_open
    cfg, sd, m = _model("w4a16")
    path = str(tmp_path / "w4.safetensors")
    save_quantized(m, path)
    with safe_open(path, framework="pt") as f:
        keys = set(f.keys())
        meta = f.metadata()
        qw = f.get_tensor("layers.1.self_attn.q_proj.qweight")
        sc = f.get_tensor("layers.1.self_attn.q_proj.scales")
        assert "layers.1.mlp.gate_proj.qweight" in keys and "lm_head.scales" in keys
        assert "layers.0.self_attn.k_norm.weight" in keys
        assert not any(k.endswith(".zeros") for k in keys)      # symmetric weights
    assert meta["format"] == "w4a16" and meta["group_size"] == "128"
    u, s = Q.quantize_w4_sym(sd["layers.1.self_attn.q_proj.weight"])
    assert torch.equal(Q.unpack_w4(qw), u) and torch.equal(sc, s)


@pytest.fixture(scope="module")
def w4_file(tmp_path_factory):
    _, _, m = _model("w4a16")
    path = str(tmp_path_factory.mktemp("ckpt") / "w4.safetensors")
    save_quantized(m, path)
    return path


@pytest.mark.parametrize("case", ["short_scales", "wrong_dtype", "missing", "group", "packing"])
def test_load_rejects_a_file_that_does_not_match_its_config(case, w4_file, tmp_path):
    """A file whose tensors or metadata disagree with its own config raises
    ValueError on load instead of reaching the kernels."""
    from safetensors import safe_open
    from safetensors.torch import save_file
    with safe_open(w4_file, framework="pt") as f:
        meta = dict(f.metadata())
        t = {k: f.get_tensor(k) for k in f.keys()}
    name = "layers.1.mlp.down_proj"
    if case == "short_scales":
        t[name + ".scales"] = t[name + ".scales"][:, :-1].contiguous()
    elif case == "wrong_dtype":
        t[name + ".qweight"] = t[name + ".qweight"].to(torch.int8)
    elif case == "missing":
        del t["layers.0.self_attn.v_proj.scales"]
    elif case == "group":
        meta["group_size"] = "64"
    else:
        meta["packing"] = "uint8 [N, K/2], high nibble = even k"
    bad = str(tmp_path / "bad.safetensors")
    save_file(t, bad, metadata=meta)
    with pytest.raises(ValueError):
        load_quantized(bad, device="cpu")


@pytest.mark.gpu
def test_loaded_w4_model_decodes_identically_on_the_gpu(tmp_path):
    """The file loaded straight onto the GPU runs the decode step to the same
    logits, bit for bit, as the model it was written from."""
    from acorninfer_amd.cache.pager import PagedCacheView
    from model_utils import feed_prompt, new_cache
    cfg = Qwen3Config.qwen3_0_6b().with_layers(2)
    sd = random_state_dict(cfg, seed=4, std=0.02, dtype=torch.float32)
    m = Qwen3DecodeModel.from_state_dict(cfg, sd, weight_format="w4a16", device="cuda")
    path = str(tmp_path / "w4.safetensors")
    save_quantized(m, path)
    r = load_quantized(path, device="cuda")
    assert r.lm_head.w.is_cuda and r.layers[0].gate_up.w.is_cuda
    prompt = [11, 4093, 77, 150000, 5]
    outs = []
    for model in (m, r):
        _, cache = new_cache(model, 8)
        outs.append(feed_prompt(model, PagedCacheView(cache), prompt))
    assert torch.equal(outs[0], outs[1])

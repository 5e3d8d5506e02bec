"""Checkpoint -> packed format converter and loader (pisceslx_amd/checkpoint.py), on the CPU.

* Known answers for the two reference quantizer states: ``_YvQuantizedLinear`` weights
  ``(q_weight - zero_point) * scale`` with per-input-column and per-tensor scales
  (model/utils/quantization.py:337-355, :494-496), and block-wise INT4 states
  ``(q - zp[b]) * scale[b]`` over flat blocks with a ragged tail (opss/quantize/methods.py:927-960).
* A two-layer reference-style checkpoint (``.pt`` with a ``model_state_dict`` wrapper as
  tools/infer/core.py:219-223 unwraps, and ``.safetensors``): both MoE layer prefixes are found;
  the converted file holds exactly what packing the layer's weights directly gives, plus the
  router keys and the shared-expert weight; converting twice gives identical bytes; a layer
  stored through the reference quantizer converts to the pack of its dequantized weights; the
  layer module loads the packed file and the whole checkpoint.
"""
import hashlib

import pytest
import torch

from pisceslx_amd import _lib
from pisceslx_amd import checkpoint as ck
from pisceslx_amd.quant import pack_experts


def test_quantized_linear_known_answers():
    q = torch.tensor([[1, -2, 127], [3, 4, -128]], dtype=torch.int8)
    scale = torch.tensor([[0.5, 0.25, 2.0]])          # per input column ([1, in]), as dim=0 gives
    zp = torch.zeros(1, 3)
    w = ck.dequantize_quantized_linear(q, scale, zp)
    assert torch.equal(w, torch.tensor([[0.5, -0.5, 254.0], [1.5, 1.0, -256.0]]))
    w = ck.dequantize_quantized_linear(q, torch.tensor(0.125), torch.tensor(-3.0))  # per tensor, asym
    assert torch.equal(w, (q.float() + 3.0) * 0.125)
    sd = {"a.q_weight": q, "a.scale": scale, "a.zero_point": zp, "b.weight": torch.ones(2, 3)}
    assert torch.equal(ck.linear_weight(sd, "a"), torch.tensor([[0.5, -0.5, 254.0], [1.5, 1.0, -256.0]]))
    assert torch.equal(ck.linear_weight(sd, "b"), torch.ones(2, 3))
    with pytest.raises(KeyError):
        ck.linear_weight(sd, "c")


def test_blockwise_int4_known_answers():
    q = torch.arange(20, dtype=torch.int32).remainder(16).view(4, 5)   # 20 codes, blocks of 8
    state = {"quantized": q, "scales": torch.tensor([0.5, 2.0, 0.25]),
             "zero_points": torch.tensor([8, 0, 15], dtype=torch.int32), "block_size": 8,
             "original_shape": torch.Size([4, 5])}
    w = ck.dequantize_blockwise_int4(state).flatten()
    flat = q.flatten().float()
    want = torch.cat([(flat[:8] - 8) * 0.5, (flat[8:16] - 0) * 2.0, (flat[16:] - 15) * 0.25])
    assert torch.equal(w, want)
    with pytest.raises(ValueError):
        ck.dequantize_blockwise_int4({**state, "scales": torch.tensor([1.0]),
                                      "zero_points": torch.tensor([0])})


H, F, E, S = 256, 384, 4, 2


def _layer_sd(prefix, g, quantized=False):
    sd = {}
    mats = []
    for i in range(E + S):
        name = f"{prefix}experts.{i}." if i < E else f"{prefix}shared_experts.{i - E}.expert."
        trio = []
        for m, shp in (("gate", (F, H)), ("up", (F, H)), ("down", (H, F))):
            w = torch.randn(*shp, generator=g) * 0.02
            if quantized:  # a YvQuantizer-style state: int8 codes, per-input-column scales
                s = (w.abs().amax(dim=0, keepdim=True) / 127).clamp(min=1e-8)
                qw = torch.clamp((w / s).round(), -128, 127).to(torch.int8)
                sd[name + f"{m}_proj.q_weight"] = qw
                sd[name + f"{m}_proj.scale"] = s
                sd[name + f"{m}_proj.zero_point"] = torch.zeros_like(s)
                w = qw.float() * s
            else:
                sd[name + f"{m}_proj.weight"] = w.to(torch.bfloat16)
                w = w.to(torch.bfloat16).float()
            trio.append(w)
        mats.append(tuple(trio))
    sd[prefix + "shared_expert_weight"] = torch.tensor([0.25, 0.75])
    sd[prefix + "router.gate.weight"] = torch.randn(E, H, generator=g)
    sd[prefix + "router.expert_bias"] = torch.randn(E, generator=g)
    return sd, mats


def _checkpoint(tmp_path, kind):
    g = torch.Generator().manual_seed(0)
    sd0, m0 = _layer_sd("model.layers.0.mlp.", g)
    sd1, m1 = _layer_sd("model.layers.1.mlp.", g, quantized=True)
    full = {**sd0, **sd1, "model.embed.weight": torch.randn(10, H, generator=g)}
    if kind == "pt":
        path = str(tmp_path / "ckpt.pt")
        torch.save({"model_state_dict": full, "step": 7}, path)
    else:
        from safetensors.torch import save_file
        path = str(tmp_path / "ckpt.safetensors")
        save_file({k: v.contiguous() for k, v in full.items()}, path)
    return path, m0, m1


def _sha(path):
    return hashlib.sha256(open(path, "rb").read()).hexdigest()


@pytest.mark.parametrize("kind", ["pt", "safetensors"])
@pytest.mark.parametrize("fmt", ["int8", "int4", "fp8", "bf16"])
def test_convert_and_load(tmp_path, kind, fmt):
    path, m0, m1 = _checkpoint(tmp_path, kind)
    assert ck.find_moe_layers(ck.StateSource(path).keys()) == ["model.layers.0.mlp.", "model.layers.1.mlp."]
    code = _lib.__dict__["W_" + fmt.upper()]
    for li, mats in ((0, m0), (1, m1)):
        dst = str(tmp_path / f"l{li}.safetensors")
        meta = ck.convert(path, dst, f"model.layers.{li}.mlp.", fmt)
        assert meta["num_routed"] == str(E) and meta["num_shared"] == str(S) and meta["format"] == fmt
        first = _sha(dst)
        ck.convert(path, dst, f"model.layers.{li}.mlp.", fmt)
        assert _sha(dst) == first                                  # deterministic
        pl = ck.load_packed(dst, device="cpu")
        want = pack_experts(mats, E, code, device="cpu")
        for n in ("w_gate", "w_up", "w_down", "s_gate", "s_up", "s_down"):
            a, b = getattr(pl.experts, n), getattr(want, n)
            assert (a is None) == (b is None), n
            if a is not None:
                assert a.dtype == b.dtype and torch.equal(a, b), n
        assert set(pl.router) == {"gate.weight", "expert_bias"}
        assert torch.equal(pl.shared_expert_weight, torch.tensor([0.25, 0.75]))


def test_load_packed_rejects_int4_scales_out_of_range(tmp_path):
    from safetensors.torch import load_file, save_file
    path, _, _ = _checkpoint(tmp_path, "safetensors")
    dst = str(tmp_path / "l0.safetensors")
    ck.convert(path, dst, "model.layers.0.mlp.", "int4")
    ck.load_packed(dst, device="cpu")
    from safetensors import safe_open
    with safe_open(dst, framework="pt", device="cpu") as f:
        meta = dict(f.metadata())
    t = load_file(dst)
    t["experts.s_down"] = t["experts.s_down"].clone()
    t["experts.s_down"].view(-1)[5] = 2.0 ** 100
    bad = str(tmp_path / "bad.safetensors")
    save_file(t, bad, metadata=meta)
    with pytest.raises(ValueError, match="experts.s_down.*outside the supported range"):
        ck.load_packed(bad, device="cpu")


def test_layer_loads_packed_and_checkpoint(tmp_path):
    from pisceslx_amd import YvDeepSeekMoELayer

    class Cfg:
        hidden_size = H
        intermediate_size = F
        moe_num_experts = E
        moe_top_k = 2
        moe_shared_experts = S

    path, m0, _ = _checkpoint(tmp_path, "pt")
    dst = str(tmp_path / "l0.safetensors")
    ck.convert(path, dst, "model.layers.0.mlp.", "int8")
    a = YvDeepSeekMoELayer(Cfg(), dtype=torch.bfloat16, weight_format="int8", router="stable")
    a.load_packed(dst)
    b = YvDeepSeekMoELayer(Cfg(), dtype=torch.bfloat16, weight_format="int8", router="stable")
    b.load_reference_checkpoint(path, "model.layers.0.mlp.")
    for n in ("w_gate", "w_up", "w_down", "s_gate", "s_up", "s_down"):
        assert torch.equal(getattr(a.experts_packed, n), getattr(b.experts_packed, n)), n
    assert torch.equal(a.router.expert_bias, b.router.expert_bias)
    assert torch.allclose(a.shared_expert_weight.float(), torch.tensor([0.25, 0.75]))
    plain = str(tmp_path / "plain.safetensors")     # a safetensors file that is not a packed layer
    ck.save_safetensors({"x": torch.zeros(2)}, plain, {"format": "int8"})
    with pytest.raises(ValueError):
        ck.load_packed(plain, device="cpu")

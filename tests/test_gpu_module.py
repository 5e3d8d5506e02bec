"""The drop-in modules on the GPU: YvDeepSeekMoELayer loaded from a reference-style state
dict, called the way YvHybridBlock calls it, against the CPU oracle — with the YvStableMoEGate
router and with the YvMoEGate router the reference's layers build (model/moe/layer.py:754-777),
including modal ids, the routing loss and the PathMoE stage cache; the stateful skip residual
across calls (model/moe/layer.py:741-753, mirrored from
tools/test/test_moe_routing_contract.py:187-201); the YvStableMoEGate contract
(tools/test/test_moe_routing_contract.py:65-81)."""
import numpy as np
import pytest
import torch

from oracle import moe_oracle
from oracle import moegate_oracle as mg
from pisceslx_amd import YvDeepSeekMoELayer, YvStableMoEGate
from pisceslx_amd import functional as yvf
from pisceslx_amd.gate import YvMoEGate

from helpers import cosine

pytestmark = pytest.mark.gpu


class Cfg:
    hidden_size = 256
    intermediate_size = 384
    moe_num_experts = 16
    moe_top_k = 4
    moe_shared_experts = 2
    moe_min_capacity = 2
    moe_fixed_shape_mode = False
    diversity_weight = 0.0


def reference_state_dict(cfg, seed=0):
    g = torch.Generator().manual_seed(seed)
    H, F, E, S = cfg.hidden_size, cfg.intermediate_size, cfg.moe_num_experts, cfg.moe_shared_experts
    r = lambda *s: torch.randn(*s, generator=g) * 0.02
    sd = {}
    for e in range(E):
        for n, shp in (("gate", (F, H)), ("up", (F, H)), ("down", (H, F))):
            sd[f"experts.{e}.{n}_proj.weight"] = r(*shp)
    for s_ in range(S):
        for n, shp in (("gate", (F, H)), ("up", (F, H)), ("down", (H, F))):
            sd[f"shared_experts.{s_}.expert.{n}_proj.weight"] = r(*shp)
    sd["shared_expert_weight"] = torch.ones(S) / S
    sd["router.gate.weight"] = r(E, H)
    sd["router.complexity_predictor.0.weight"] = r(64, H)
    sd["router.complexity_predictor.0.bias"] = torch.zeros(64)
    sd["router.complexity_predictor.2.weight"] = r(1, 64)
    sd["router.complexity_predictor.2.bias"] = torch.zeros(1)
    return sd


def oracle_params_of(layer):
    cpu = layer.experts_packed.to("cpu")
    pred = layer.router.complexity_predictor
    return moe_oracle.LayerParams(
        hidden=layer.hidden_size, ffn=layer.intermediate_size, num_experts=layer.num_experts,
        num_shared=layer.num_shared_experts, top_k=layer.top_k,
        gate_weight=layer.router.gate.weight.detach().cpu(),
        pred=(pred[0].weight.detach().cpu(), pred[0].bias.detach().cpu(),
              pred[2].weight.detach().cpu(), pred[2].bias.detach().cpu()),
        bias=None, fixed_shape_mode=False, dynamic_capacity=True,
        capacity_factor=1.0, min_capacity=layer.router.min_capacity,
        mix_param=layer.shared_expert_weight.detach().cpu(),
        expert_fn=lambda i: cpu.dequantize(i, torch.float32))


def _oracle_call(layer, x, skip):
    x2d = x.reshape(-1, x.shape[-1])
    st = layer.router.router_state(yvf._act(x2d.dtype))
    lg = yvf.router_logits(x2d.contiguous(), st)[:, :layer.num_experts].cpu().numpy()
    cap = int(layer.last_routing.capacity.item())
    o = moe_oracle.layer_forward(x2d.cpu(), oracle_params_of(layer), logits=lg, cap=cap,
                                 skip=None if skip is None else skip.reshape(x2d.shape).cpu())
    assert cap == moe_oracle.layer_capacity(oracle_params_of(layer), x2d.cpu())
    return o


@pytest.mark.parametrize("fmt", ["int8", "bf16"])
def test_deepseek_layer_drop_in(cuda, oracle, fmt):
    cfg = Cfg()
    layer = YvDeepSeekMoELayer(cfg, device=cuda, dtype=torch.bfloat16, weight_format=fmt,
                               router="stable").eval()
    layer.load_reference_state_dict(reference_state_dict(cfg))
    g = torch.Generator(device=cuda).manual_seed(1)
    x1 = torch.randn(2, 17, cfg.hidden_size, device=cuda, generator=g).to(torch.bfloat16)
    x2 = torch.randn(2, 17, cfg.hidden_size, device=cuda, generator=g).to(torch.bfloat16)
    x3 = torch.randn(1, 9, cfg.hidden_size, device=cuda, generator=g).to(torch.bfloat16)

    print(f"module drop-in fmt={fmt}", flush=True)
    out1, loss = layer(x1, modal_id=torch.zeros(2, dtype=torch.long, device=cuda))
    torch.cuda.synchronize()
    assert out1.shape == x1.shape and float(loss) == 0.0
    out1 = out1.reshape(-1, cfg.hidden_size)
    o1 = _oracle_call(layer, x1, None)
    assert cosine(out1.cpu(), o1["out"]) >= 0.9999
    assert float((out1.cpu().double() - o1["out"].double()).abs().max()) <= 2e-2
    skip1 = layer._skip_buffer.clone()

    out2, _ = layer(x2)                     # same shape: adds 0.1 * previous shared output
    torch.cuda.synchronize()
    out2 = out2.reshape(-1, cfg.hidden_size)
    o2 = _oracle_call(layer, x2, skip1)
    assert cosine(out2.cpu(), o2["out"]) >= 0.9999
    assert float((out2.cpu().double() - o2["out"].double()).abs().max()) <= 2e-2
    no_skip = _oracle_call(layer, x2, None)["out"]
    assert float((out2.cpu().float() - no_skip.float()).abs().max()) > 1e-3  # the residual is there

    out3, _ = layer(x3)                     # shape change: no residual from the 2x17 batch
    torch.cuda.synchronize()
    assert out3.shape == x3.shape
    out3 = out3.reshape(-1, cfg.hidden_size)
    o3 = _oracle_call(layer, x3, None)
    assert cosine(out3.cpu(), o3["out"]) >= 0.9999


def test_stable_gate_contract(cuda, oracle):
    gate = YvStableMoEGate(hidden_size=64, num_experts=4, top_k=2, capacity_factor=1.0,
                           min_capacity=1, device=cuda).eval()
    x = torch.randn(1, 24, 64, device=cuda)
    weights, indices, loss = gate(x)
    torch.cuda.synchronize()
    assert weights.shape == (24, 2) and indices.shape == (24, 2)
    assert indices.dtype == torch.int64 and float(loss) == 0.0
    tot = weights.sum(-1)
    assert bool(torch.all((tot <= 1.0 + 1e-5) | (tot == 0))) and bool(torch.all(weights >= 0))
    with pytest.raises(NotImplementedError):
        gate.train()(x)


@pytest.mark.parametrize("load_records", [4, 23])
def test_stable_gate_load_adjustment_routing(cuda, oracle, load_records):
    """A gate whose routing history is non-empty (gate.py:1192-1204): the adjustment
    0.1 * (predicted - recent) is added to the logits before the softmax. Uniform prediction
    below 10 load records, the LSTM's from 10 on. The GPU routing must equal the oracle's
    routing of the GPU's fp32 logits with that bias, bit for bit, and differ from the routing
    without it."""
    E, H, k = 16, 256, 4
    torch.manual_seed(3)
    gate = YvStableMoEGate(H, E, top_k=k, min_capacity=2, device=cuda).eval()
    rng = np.random.default_rng(load_records)
    rows = rng.dirichlet(np.full(E, 0.8), size=6)          # skewed but above the 0.7 ratio
    recent = rows.mean(0)
    assert -(recent * np.log(recent)).sum() / np.log(E) > 0.75
    with torch.no_grad():
        gate.gate.weight.normal_(0.0, 0.02)
        gate.routing_history[:6] = torch.tensor(rows, dtype=torch.float32)
        gate.history_ptr.fill_(6)
        gate.expert_load_buffer[:load_records] = torch.tensor(
            rng.dirichlet(np.ones(E), size=load_records), dtype=torch.float32)
        gate.load_buffer_ptr.fill_(load_records)
        for p_ in gate.predictor_head.parameters():
            p_.normal_(0.0, 2.0)                           # a prediction far from uniform
    x = torch.randn(1, 96, H, device=cuda)
    print(f"stable gate load adjustment, {load_records} load records", flush=True)
    weights, indices, _ = gate(x)
    adj = gate._load_adjustment()
    assert adj is not None
    st = gate.router_state(yvf._act(x.dtype))
    assert st.bias is adj
    lg = yvf.router_logits(x.reshape(-1, H).contiguous(), st)
    torch.cuda.synchronize()
    params = moe_oracle.LayerParams(
        hidden=H, ffn=64, num_experts=E, num_shared=0, top_k=k,
        gate_weight=gate.gate.weight.detach().cpu(),
        pred=tuple(t.detach().cpu() for t in (gate.complexity_predictor[0].weight,
                                              gate.complexity_predictor[0].bias,
                                              gate.complexity_predictor[2].weight,
                                              gate.complexity_predictor[2].bias)),
        bias=None, fixed_shape_mode=False, dynamic_capacity=True, capacity_factor=1.0,
        min_capacity=2, mix_param=None, expert_fn=None)
    cap = moe_oracle.layer_capacity(params, x.reshape(-1, H).cpu())
    lgn = lg[:, :E].cpu().numpy()
    r = oracle.route(lgn, k, cap, adj.cpu().numpy())
    assert np.array_equal(indices.cpu().numpy(), r.indices.astype(np.int64))
    assert np.array_equal(weights.cpu().numpy().view(np.uint32), r.weights.view(np.uint32))
    r0 = oracle.route(lgn, k, cap, None)
    assert not np.array_equal(r0.indices, r.indices)       # the bias changed some choices


def test_layer_rejects_training_mode(cuda):
    layer = YvDeepSeekMoELayer(Cfg(), device=cuda, dtype=torch.bfloat16, weight_format="bf16")
    with pytest.raises(NotImplementedError):
        layer.train()(torch.randn(1, 4, Cfg.hidden_size, device=cuda).to(torch.bfloat16))


def moegate_state_dict(cfg, seed=1):
    """router.* keys of a YvMoEGate (its own initialisation, then a few buffers and the
    affinity made non-trivial), with graph-builder / importance keys the module skips."""
    torch.manual_seed(seed)
    g = YvMoEGate(cfg.hidden_size, cfg.moe_num_experts, top_k=cfg.moe_top_k, dtype=torch.bfloat16,
                  cfg=cfg)
    with torch.no_grad():
        g.expert_modal_affinity.normal_(0.0, 0.3)
        g.expert_bias.normal_(0.0, 0.2)
        g.hicl_dg_encoder.dg_bias.normal_(0.0, 0.05)
        for name in ("w_hicl", "w_got", "w_soft", "w_expert_orient"):
            getattr(g, name).fill_(0.5)
    sd = {"router." + k: v for k, v in g.state_dict().items()}
    sd["router.got_graph_builder.q_proj.weight"] = torch.zeros(cfg.hidden_size, cfg.hidden_size)
    sd["router.importance_proj.0.weight"] = torch.zeros(cfg.hidden_size // 4, cfg.hidden_size)
    return sd


def _moegate_oracle_check(layer, x, oracle, skip, modal_id=None, route_logits=None):
    """GPU logits vs float64, routing bit-exact given the routed logits, output vs the oracle
    layer on those logits, loss vs the oracle's."""
    g = layer.router
    x2d = x.reshape(-1, x.shape[-1])
    p = mg.params_from_state_dict(g.state_dict(), torch.bfloat16, soft_temperature=g.soft_moe_temperature)
    og = mg.moegate_forward(x.cpu(), p, layer.top_k, modal_id=None if modal_id is None else modal_id.cpu())
    lg = g.last_logits.cpu().numpy()
    ref = og["logits"].numpy()
    assert float(np.abs(lg - ref).max()) <= 1e-4 * max(1.0, float(np.abs(ref).max()))
    assert float(g._last_loss_f32) == pytest.approx(og["loss"], rel=1e-4, abs=1e-7)
    routed = lg if route_logits is None else route_logits
    r = oracle.route(routed.astype(np.float32), layer.top_k, -1, None)
    assert np.array_equal(layer.last_routing.indices.cpu().numpy(), r.indices.astype(np.int64))
    assert np.array_equal(layer.last_routing.perm.cpu().numpy(), r.perm)
    cpu = layer.experts_packed.to("cpu")
    params = moe_oracle.LayerParams(
        hidden=layer.hidden_size, ffn=layer.intermediate_size, num_experts=layer.num_experts,
        num_shared=layer.num_shared_experts, top_k=layer.top_k,
        gate_weight=torch.zeros(layer.num_experts, layer.hidden_size), pred=None, bias=None,
        fixed_shape_mode=True, dynamic_capacity=False, capacity_factor=1.0, min_capacity=0,
        mix_param=None if layer.shared_expert_weight is None else layer.shared_expert_weight.detach().cpu(),
        expert_fn=lambda i: cpu.dequantize(i, torch.float32))
    return moe_oracle.layer_forward(x2d.cpu(), params, logits=routed, cap=-1,
                                    skip=None if skip is None else skip.reshape(x2d.shape).cpu())


def test_deepseek_layer_moegate_router(cuda, oracle):
    cfg = Cfg()
    layer = YvDeepSeekMoELayer(cfg, device=cuda, dtype=torch.bfloat16, weight_format="int8").eval()
    assert isinstance(layer.router, YvMoEGate)
    sd = reference_state_dict(cfg)
    sd = {k: v for k, v in sd.items() if not k.startswith("router.")}
    sd.update(moegate_state_dict(cfg))
    layer.load_reference_state_dict(sd, strict=True)
    layer.router._path_moe_stage_size = 1
    gen = torch.Generator(device=cuda).manual_seed(2)
    x1 = torch.randn(3, 11, cfg.hidden_size, device=cuda, generator=gen).to(torch.bfloat16)
    x2 = torch.randn(3, 11, cfg.hidden_size, device=cuda, generator=gen).to(torch.bfloat16)
    modal = torch.tensor([1, 4, 0], device=cuda)
    print("module moegate router", flush=True)
    out1, loss1 = layer(x1, modal_id=modal)
    torch.cuda.synchronize()
    o1 = _moegate_oracle_check(layer, x1, oracle, None, modal_id=modal)
    out1 = out1.reshape(-1, cfg.hidden_size).cpu()
    assert cosine(out1, o1["out"]) >= 0.9999
    assert float((out1.double() - o1["out"].double()).abs().max()) <= 2e-2
    assert loss1.dtype == torch.bfloat16 and float(loss1) > 0
    skip1 = layer._skip_buffer.clone()
    out2, _ = layer(x2)                     # skip residual from call 1
    torch.cuda.synchronize()
    o2 = _moegate_oracle_check(layer, x2, oracle, skip1)
    out2 = out2.reshape(-1, cfg.hidden_size).cpu()
    assert cosine(out2, o2["out"]) >= 0.9999
    assert float((out2.double() - o2["out"].double()).abs().max()) <= 2e-2


def test_moegate_layer_path_moe_stage(cuda, oracle):
    cfg = Cfg()
    cfg.moe_shared_experts = 0
    layer = YvDeepSeekMoELayer(cfg, device=cuda, dtype=torch.bfloat16, weight_format="bf16").eval()
    sd = reference_state_dict(cfg)
    sd = {k: v for k, v in sd.items() if not k.startswith("router.")}
    sd.update(moegate_state_dict(cfg, seed=5))
    layer.load_reference_state_dict(sd, strict=True)
    assert layer.router._path_moe_stage_size == 4
    gen = torch.Generator(device=cuda).manual_seed(3)
    xs = [torch.randn(2, 8, cfg.hidden_size, device=cuda, generator=gen).to(torch.bfloat16)
          for _ in range(5)]
    first_logits = None
    for i, x in enumerate(xs):
        out, loss = layer(x)
        torch.cuda.synchronize()
        lg = layer.router.last_logits.cpu().numpy()
        if i % 4 == 0:
            first_logits = lg               # a stage starts: routes on its own logits
            o = _moegate_oracle_check(layer, x, oracle, None)
        else:                               # later calls route on the stage's first logits
            o = _moegate_oracle_check(layer, x, oracle, None, route_logits=first_logits)
        got = out.reshape(-1, cfg.hidden_size).cpu()
        assert cosine(got, o["out"]) >= 0.9999, i


def test_layer_from_packed_checkpoint(cuda, tmp_path):
    """A reference checkpoint converted offline and loaded gives the same forward as the layer
    loaded from the state dict directly (same packed bytes)."""
    from pisceslx_amd import checkpoint as ck
    cfg = Cfg()
    sd = {"layers.0.mlp." + k: v for k, v in reference_state_dict(cfg, seed=4).items()}
    src = str(tmp_path / "model.pt")
    torch.save({"model": sd}, src)
    dst = str(tmp_path / "layer0.safetensors")
    ck.convert(src, dst, "layers.0.mlp.", "int8")
    a = YvDeepSeekMoELayer(cfg, device=cuda, dtype=torch.bfloat16, weight_format="int8",
                           router="stable").eval()
    a.load_packed(dst)
    b = YvDeepSeekMoELayer(cfg, device=cuda, dtype=torch.bfloat16, weight_format="int8",
                           router="stable").eval()
    b.load_reference_state_dict(reference_state_dict(cfg, seed=4))
    x = torch.randn(2, 13, cfg.hidden_size, device=cuda,
                    generator=torch.Generator(device=cuda).manual_seed(5)).to(torch.bfloat16)
    print("packed checkpoint layer", flush=True)
    oa, _ = a(x)
    ob, _ = b(x)
    torch.cuda.synchronize()
    assert torch.equal(oa, ob)


def _reference_quantized(w, symmetric):
    """A ``_YvQuantizedLinear`` state of ``w`` as ``YvQuantizer.quantize_tensor`` builds it
    (model/utils/quantization.py:336-355): int8 codes, per-input-column scale [1, in] (amax over
    dim 0 / 127), zero point 0 (symmetric) or round(-128 - min / scale) (asymmetric)."""
    scale = (w.abs().amax(dim=0, keepdim=True) / 127).clamp(min=1e-8)
    zp = torch.zeros_like(scale) if symmetric else \
        (-128 - w.amin(dim=0, keepdim=True) / scale).round().clamp(-128, 127)
    q = torch.clamp((w / scale + zp).round(), -128, 127).to(torch.int8)
    return q, scale, zp


@pytest.mark.parametrize("fmt", ["int8", "bf16"])
def test_layer_from_reference_quantized_checkpoint(cuda, oracle, tmp_path, fmt):
    """A checkpoint whose experts the reference quantizer stored (``q_weight``/``scale``/
    ``zero_point``; routed experts symmetric, shared experts asymmetric), converted and loaded,
    run through the GPU layer and compared with the oracle on the checkpoint's own dequantized
    weights ``(q_weight - zero_point) * scale`` — the weights the reference's forward uses
    (model/utils/quantization.py:494-496).

    bf16 keeps those weights to bf16 rounding: the layer tolerance holds. int8 stores one scale
    per output channel, so weights quantized per input column are quantized again; that costs a
    measured cosine of 0.99990 on this layer (1.4 % relative error), bounded here at 0.9997.
    Against the oracle on the packed (converted) weights both formats meet the layer tolerance.
    """
    from pisceslx_amd import checkpoint as ck
    cfg = Cfg()
    full = reference_state_dict(cfg, seed=6)
    sd, deq = {}, {}
    for key, v in full.items():
        if key.endswith("_proj.weight"):
            name = key[:-len(".weight")]
            q, s, zp = _reference_quantized(v, symmetric=not key.startswith("shared_"))
            sd[f"model.layers.2.mlp.{name}.q_weight"] = q
            sd[f"model.layers.2.mlp.{name}.scale"] = s
            sd[f"model.layers.2.mlp.{name}.zero_point"] = zp
            deq[name] = (q.float() - zp) * s
        else:
            sd["model.layers.2.mlp." + key] = v
    src = str(tmp_path / "quantized.pt")
    torch.save({"model_state_dict": sd}, src)
    dst = str(tmp_path / "layer2.safetensors")
    ck.convert(src, dst, "model.layers.2.mlp.", fmt)
    layer = YvDeepSeekMoELayer(cfg, device=cuda, dtype=torch.bfloat16, weight_format=fmt,
                               router="stable").eval()
    layer.load_packed(dst)
    x = torch.randn(3, 21, cfg.hidden_size, device=cuda,
                    generator=torch.Generator(device=cuda).manual_seed(8)).to(torch.bfloat16)
    print(f"reference-quantized checkpoint fmt={fmt}", flush=True)
    out, _ = layer(x)
    torch.cuda.synchronize()
    got = out.reshape(-1, cfg.hidden_size).cpu()

    packed = _oracle_call(layer, x, None)           # oracle on the converted weights
    assert cosine(got, packed["out"]) >= 0.9999
    assert float((got.double() - packed["out"].double()).abs().max()) <= 2e-2

    E = cfg.moe_num_experts
    name = lambda i, m: (f"experts.{i}.{m}_proj" if i < E
                         else f"shared_experts.{i - E}.expert.{m}_proj")
    p = oracle_params_of(layer)
    p.expert_fn = lambda i: tuple(deq[name(i, m)] for m in ("gate", "up", "down"))
    x2d = x.reshape(-1, cfg.hidden_size)
    ref = moe_oracle.layer_forward(x2d.cpu(), p, routing=packed["routing"])
    c = cosine(got, ref["out"])
    print(f"  vs dequantized checkpoint weights: cos {c:.6f}", flush=True)
    if fmt == "bf16":
        assert c >= 0.9999
        assert float((got.double() - ref["out"].double()).abs().max()) <= 2e-2
    else:
        assert c >= 0.9997

"""RMSNorm of the MoE input on the GPU (yvmoe_rmsnorm) against the CPU oracle
(oracle/norm_oracle.py, the fused_rms_norm semantics of opss/kernels/fused_rms_norm.py:42).

bf16: one norm without bias within one bf16 ulp of the float64 oracle (the kernel sums in
fp32) and at least 99% identical; with a bias or a second norm, within two ulps of the
largest magnitude the roundings saw before the bias adds (a one-ulp difference of an earlier
rounding carries through a bias add that cancels); fp32: 1e-5 of that magnitude. Cases: the hidden sizes of the layer
configurations (4096, 5120, 7168) and small ones, rows longer than the register-resident
form (16384, 12288 bf16; 8192 fp32: the intermediate norm goes through the output), four
wavefronts per row (under 2048 rows) and one (2048 rows and more), bias,
two norms in one pass (YvHybridBlock's norm_fusion then norm_mlp), in place, zero rows,
scales 1e-4..1e4, N = 0, argument errors; the YvRMSNorm module and the MoE half of the
hybrid block loaded from block-style state dict keys.
"""
import pytest
import torch

from oracle import norm_oracle as no
from pisceslx_amd import YvHybridBlockMLP, YvRMSNorm
from pisceslx_amd import _lib
from pisceslx_amd import functional as yvf

pytestmark = pytest.mark.gpu


def _norm(H, dtype, seed, bias=False, eps=1e-6):
    g = torch.Generator().manual_seed(seed)
    w = (1.0 + 0.3 * torch.randn(H, generator=g)).to(dtype)
    b = (0.1 * torch.randn(H, generator=g)).to(dtype) if bias else None
    return w, b, eps


def _bf16_ulp(mag):
    """Spacing of bf16 values at magnitude mag (8 significand bits)."""
    e = torch.floor(torch.log2(mag.clamp_min(2.0 ** -126)))
    return torch.pow(2.0, e - 7)


def _magnitude(x, norms):
    """Per element, the largest magnitude the last rounding's inputs had: the normalised value
    before its bias, the bias, and the first norm's own pre-add magnitude carried through the
    second norm's scaling (w2 / rms2). A one-ulp difference at that magnitude survives a bias
    add that cancels (y + b close to 0)."""
    xd = x.to(torch.float64)
    mag = None
    y = x
    for w, b, eps in norms:
        if mag is not None:
            yd = y.to(torch.float64)
            rms = torch.sqrt((yd * yd).mean(-1, keepdim=True) + eps)
            mag = mag * w.to(torch.float64).abs() / rms
        pre = no.rms_norm_once(y, w, None, eps, torch.float64).abs()
        m = pre if b is None else torch.maximum(pre, b.to(torch.float64).abs())
        mag = m if mag is None else torch.maximum(mag, m)
        y = no.rms_norm_once(y, w, b, eps, x.dtype)
    del xd
    return mag


def _compare(got, want, norms, x):
    """One norm without bias: within one bf16 ulp of the oracle (fp32: 1e-5 relative). With a
    bias or a second norm: within two ulps (fp32: 1e-5) of the magnitude the roundings had
    before the bias adds."""
    got = got.cpu()
    single = len(norms) == 1 and norms[0][1] is None
    if got.dtype == torch.bfloat16:
        d = no.bf16_ulp_distance(got, want)
        same = float((d == 0).float().mean()) if d.numel() else 1.0
        print(f"  max ulp {int(d.max()) if d.numel() else 0}, identical {same:.5f}", flush=True)
        if d.numel() == 0:
            return
        assert same >= 0.99
        if single:
            assert int(d.max()) <= 1
        else:
            mag = torch.maximum(want.to(torch.float64).abs(), _magnitude(x, norms))
            err = (got.to(torch.float64) - want.to(torch.float64)).abs()
            assert bool((err <= 2 * _bf16_ulp(mag)).all()), float((err / _bf16_ulp(mag)).max())
    else:
        ref = want.to(torch.float64)
        err = (got.to(torch.float64) - ref).abs()
        mag = ref.abs() if single else torch.maximum(ref.abs(), _magnitude(x, norms))
        print(f"  max rel {float((err / mag.clamp_min(1e-30)).max()) if err.numel() else 0:.3e}",
              flush=True)
        assert err.numel() == 0 or bool((err <= 1e-5 * mag.clamp_min(1e-30)).all())


@pytest.mark.parametrize("N,H,dtype,nn,bias", [
    (64, 4096, torch.bfloat16, 1, False),
    (64, 4096, torch.bfloat16, 2, False),
    (333, 5120, torch.bfloat16, 2, True),
    (7, 7168, torch.bfloat16, 1, True),
    (5, 8, torch.bfloat16, 2, False),
    (9, 8192, torch.bfloat16, 2, False),
    (6, 16384, torch.bfloat16, 2, True),
    (3, 12288, torch.bfloat16, 1, False),
    (50, 4096, torch.float32, 2, True),
    (4, 8192, torch.float32, 2, False),
    (1, 24, torch.float32, 1, False),
    # 2048 rows and more: two wavefronts per row instead of four
    (2100, 4096, torch.bfloat16, 2, False),
    (2048, 5120, torch.bfloat16, 1, True),
    (2050, 12288, torch.bfloat16, 2, True),
    (2049, 2048, torch.float32, 2, True),
    (2049, 4096, torch.bfloat16, 2, False),   # odd count: the last work-group has a dead row
    (2051, 16384, torch.bfloat16, 2, True),   # the same, rows longer than the registers hold
])
def test_rmsnorm_matches_oracle(cuda, N, H, dtype, nn, bias):
    print(f"rmsnorm N={N} H={H} dtype={dtype} norms={nn} bias={bias}", flush=True)
    g = torch.Generator().manual_seed(N * 31 + H)
    x = (torch.randn(N, H, generator=g) * torch.logspace(-4, 4, N).unsqueeze(1)).to(dtype)
    if N > 2:
        x[1].zero_()                                # a zero row: eps keeps it finite (0 out)
    norms = [_norm(H, dtype, seed=i + H, bias=bias) for i in range(nn)]
    want = no.rms_norm(x, norms)
    xg = x.cuda()
    got = yvf.rms_norm(xg, [(w.cuda(), None if b is None else b.cuda(), e) for w, b, e in norms])
    torch.cuda.synchronize()
    _compare(got, want, norms, x)
    assert torch.equal(xg.cpu(), x)                 # input untouched
    # in place gives the same bits
    yvf.rms_norm(xg, [(w.cuda(), None if b is None else b.cuda(), e) for w, b, e in norms], out=xg)
    torch.cuda.synchronize()
    assert torch.equal(xg, got)


def test_rmsnorm_empty_and_errors(cuda):
    w = torch.ones(64, dtype=torch.bfloat16, device=cuda)
    y = yvf.rms_norm(torch.zeros(0, 64, dtype=torch.bfloat16, device=cuda), [(w, None, 1e-6)])
    assert y.shape == (0, 64)
    x = torch.randn(4, 64, device=cuda).to(torch.bfloat16)
    with pytest.raises(ValueError):
        yvf.rms_norm(x, [(w.float(), None, 1e-6)])           # weight dtype must match
    with pytest.raises(ValueError):
        yvf.rms_norm(x, [(w, None, 1e-6)] * 3)              # one or two norms
    with pytest.raises(ValueError, match="multiple of 8"):
        yvf.rms_norm(torch.randn(4, 60, device=cuda).to(torch.bfloat16),
                     [(torch.ones(60, dtype=torch.bfloat16, device=cuda), None, 1e-6)])
    with pytest.raises(ValueError, match="eps"):
        yvf.rms_norm(x, [(w, None, -1.0)])
    p = (_lib.RMSNormParams * 1)()
    p[0].weight = w.data_ptr() + 2                          # misaligned weight
    p[0].eps = 1e-6
    rc = _lib.lib().yvmoe_rmsnorm(x.data_ptr(), _lib.ACT_BF16, 4, 64, p, 1, x.data_ptr(), None)
    assert rc == _lib.YVMOE_ERR_ARG


def test_yvrmsnorm_module(cuda):
    H = 4096
    m = YvRMSNorm(H, use_bias=True, device=cuda, dtype=torch.bfloat16)
    with torch.no_grad():
        m.weight.normal_(1.0, 0.2)
        m.bias.normal_(0.0, 0.05)
    x = torch.randn(3, 11, H, device=cuda).to(torch.bfloat16)
    y = m(x)
    torch.cuda.synchronize()
    assert y.shape == x.shape and y.dtype == x.dtype
    norms = [(m.weight.detach().cpu(), m.bias.detach().cpu(), 1e-6)]
    want = no.rms_norm(x.cpu().reshape(-1, H), norms)
    _compare(y.reshape(-1, H), want, norms, x.cpu().reshape(-1, H))
    assert m.state_dict().keys() == {"weight", "bias"}


class BlockCfg:
    hidden_size = 256
    intermediate_size = 384
    moe_num_experts = 16
    moe_top_k = 4
    moe_shared_experts = 1
    moe_min_capacity = 2
    moe_fixed_shape_mode = False
    diversity_weight = 0.0
    n_layer = 4


def test_hybrid_block_mlp(cuda):
    cfg = BlockCfg()
    blk = YvHybridBlockMLP(cfg, device=cuda, dtype=torch.bfloat16, router="stable").eval()
    H = cfg.hidden_size
    g = torch.Generator().manual_seed(3)
    sd = {k: v.detach().cpu().clone() for k, v in blk.state_dict().items()}
    sd["norm_fusion.weight"] = (1.0 + 0.2 * torch.randn(H, generator=g)).to(torch.bfloat16)
    sd["norm_mlp.weight"] = (1.0 + 0.2 * torch.randn(H, generator=g)).to(torch.bfloat16)
    sd["residual_scale_mlp"] = torch.tensor([0.3535534], dtype=torch.bfloat16)
    blk.load_state_dict(sd, strict=False)
    assert float(blk.residual_scale_mlp) == float(torch.tensor(0.3535534).to(torch.bfloat16))
    h = (torch.randn(2, 9, H, generator=g) * 3).to(torch.bfloat16).cuda()
    out, aux = blk(h)
    torch.cuda.synchronize()
    # the two norms, checked against the oracle; then the layer and the residual composed
    norms = [(sd["norm_fusion.weight"], None, 1e-6), (sd["norm_mlp.weight"], None, 1e-6)]
    xn = no.rms_norm(h.cpu().reshape(-1, H), norms)
    xg = yvf.rms_norm(h.reshape(-1, H), [(blk.norm_fusion.weight.detach(), None, 1e-6),
                                         (blk.norm_mlp.weight.detach(), None, 1e-6)])
    _compare(xg, xn, norms, h.cpu().reshape(-1, H))
    blk.mlp._skip_buffer = None                     # the same (empty) skip state as blk(h) saw
    mlp_out, _ = blk.mlp(xg.reshape(h.shape))
    want = h + blk.residual_scale_mlp * mlp_out
    assert out.shape == h.shape and torch.equal(out, want) and aux.numel() == 1

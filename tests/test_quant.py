"""Weight formats (pisceslx_amd/quant.py) against their closed forms, on the CPU.

int8 per output channel (YvQuantizer.quantize_tensor arithmetic, model/utils/quantization.py:
337-355), int4 group-128 with zero point 8 and low-nibble-first packing (kv_cache.py:245),
fp8 e4m3fn with 128x128 block scales (quantize_to_fp8, opss/quantize/engine.py:841-883), and
the three-term bf16 split of the fp32 predictor weight used by the router GEMM.
"""
import numpy as np
import pytest
import torch

from pisceslx_amd import _lib
from pisceslx_amd import quant


def test_int8_round_trip_error_and_scale():
    g = torch.Generator().manual_seed(0)
    w = torch.randn(64, 256, generator=g) * 0.02
    w[3] = 0.0
    q, s = quant.quantize_int8(w)
    assert q.dtype == torch.int8 and s.dtype == torch.bfloat16 and s.shape == (64,)
    amax = w.abs().amax(1)
    torch.testing.assert_close(s.float(), (amax / 127).clamp(min=1e-8).to(torch.bfloat16).float())
    d = quant.dequantize_int8(q, s)
    assert (d - w).abs().le(s.float()[:, None] / 2 + 1e-12).all()
    assert (q[3] == 0).all() and (d[3] == 0).all()
    # the largest element maps to +-127 (or its neighbour through the bf16 scale rounding)
    top = q.int().abs().amax(1)[torch.arange(64) != 3]
    assert top.ge(126).all() and top.le(128).all()


def test_int4_packing_order_and_groups():
    w = torch.zeros(2, 256)
    codes = torch.tensor([1 + (i * 7) % 15 for i in range(256)], dtype=torch.float32)  # 1..15
    s_true = 0.01
    w[0] = (codes - 8) * s_true
    w[0, 0] = 7 * s_true   # make |max| of group 0 exactly 7 s (code 15)
    w[0, 128] = -7 * s_true
    packed, s = quant.quantize_int4(w)
    assert packed.shape == (2, 128) and s.shape == (2, 2)
    un = quant.unpack_int4(packed)
    assert torch.equal(un[:, 0::2], packed & 0xF) and torch.equal(un[:, 1::2], packed >> 4)
    d = quant.dequantize_int4(packed, s)
    assert (d[0] - w[0]).abs().max() <= s.float()[0].max() / 2 + 1e-7
    assert (un[1] == 8).all() and (d[1] == 0).all()          # all-zero row: code 8, value 0
    assert un[0, 0] == 15 and un[0, 128] == 1                  # +-absmax -> +-7 around 8


def test_int4_scale_range_edges():
    """The kernels apply an int4 group scale exactly for bf16 2^-126 <= |s| < 2^97 (and 0):
    the quantizer and the packed-file loader reject scales outside that range."""
    top = 2.0 ** 97 - 2.0 ** 89            # the largest bf16 below 2^97
    w = torch.zeros(1, 128)
    w[0, 0] = 7 * top
    _, s = quant.quantize_int4(w)
    assert float(s[0, 0]) == top
    w[0, 0] = 7 * 2.0 ** 97
    with pytest.raises(ValueError, match="outside the supported range"):
        quant.quantize_int4(w)
    ok = torch.tensor([0.0, 2.0 ** -126, -(2.0 ** -126), top, -top, 1e-8], dtype=torch.bfloat16)
    quant.check_int4_scales(ok)
    for bad in (2.0 ** 97, -(2.0 ** 97), 2.0 ** -127, -(2.0 ** -130), float("inf"), float("nan")):
        with pytest.raises(ValueError, match="outside the supported range"):
            quant.check_int4_scales(torch.tensor([0.5, bad], dtype=torch.bfloat16))


def test_fp8_blocks_exact_and_clamped():
    g = torch.Generator().manual_seed(1)
    w = torch.randn(256, 384, generator=g) * 0.05
    q, s = quant.quantize_fp8(w)
    assert q.dtype == torch.uint8 and s.shape == (2, 3)
    blocks = w.view(2, 128, 3, 128).abs().amax(dim=(1, 3))
    torch.testing.assert_close(s, blocks / 448.0)
    v = q.view(torch.float8_e4m3fn).float()
    assert v.abs().max() <= 448.0
    # each block's absmax element quantizes to exactly +-448
    for bi in range(2):
        for bj in range(3):
            blk = v[bi * 128:(bi + 1) * 128, bj * 128:(bj + 1) * 128]
            assert blk.abs().max() == 448.0
    d = quant.dequantize_fp8(q, s)
    rel = ((d - w).abs() / w.abs().clamp(min=1e-3)).max()
    assert rel < 0.07  # e4m3 has 3 mantissa bits: half-ulp relative error 1/16


def test_router_split_is_exact_to_one_ulp():
    g = torch.Generator().manual_seed(2)
    w1 = torch.randn(64, 512, generator=g) * 0.02
    hi, mid, lo = quant.split_bf16x3(w1)
    recon = hi.double() + mid.double() + lo.double()
    ulp = torch.abs(w1.double()) * 2.0 ** -23
    assert ((recon - w1.double()).abs() <= ulp + 1e-45).all()
    wr = quant.pack_router(torch.randn(10, 512, generator=g).to(torch.bfloat16), w1, _lib.ACT_BF16)
    assert wr.shape == (16 + 192, 512)
    wr = quant.unblock_matrix(wr, _lib.W_BF16)                 # stored in the blocked order
    assert (wr[10:16] == 0).all() and torch.equal(wr[16:80], hi) and torch.equal(wr[144:], lo)
    wr32 = quant.pack_router(torch.randn(10, 512, generator=g), w1, _lib.ACT_F32)
    assert wr32.shape == (16 + 64, 512) and torch.equal(wr32[16:], w1)


@pytest.mark.parametrize("fmt", [_lib.W_F32, _lib.W_BF16, _lib.W_INT8, _lib.W_INT4, _lib.W_FP8])
def test_packer_dequantize_matches_formats(fmt):
    g = torch.Generator().manual_seed(3)
    ws = [(torch.randn(256, 128, generator=g) * 0.02, torch.randn(256, 128, generator=g) * 0.02,
           torch.randn(128, 256, generator=g) * 0.02) for _ in range(3)]
    pk = quant.pack_experts(ws, 2, fmt, device="cpu")
    assert pk.num_routed == 2 and pk.num_shared == 1
    for i, (wg, wu, wd) in enumerate(ws):
        dg, du, dd = pk.dequantize(i)
        for a, b in ((dg, wg), (du, wu), (dd, wd)):
            if fmt == _lib.W_F32:
                bound = torch.zeros_like(b)
            elif fmt == _lib.W_BF16:
                bound = b.abs() * 2.0 ** -8                                   # half a bf16 ulp
            elif fmt == _lib.W_INT8:
                bound = (b.abs().amax(1, keepdim=True) / 127) * (0.5 + 2.0 ** -7)
            elif fmt == _lib.W_INT4:
                grp = b.abs().view(b.shape[0], -1, 128).amax(-1, keepdim=True) / 7
                bound = (grp * (0.5 + 2.0 ** -6)).expand(-1, -1, 128).reshape(b.shape)
            else:
                bound = b.abs() / 16 + 1e-6                                   # e4m3: 3 mantissa bits
            assert ((a - b).abs() <= bound + 1e-9).all()


@pytest.mark.parametrize("fmt", [_lib.W_BF16, _lib.W_INT8, _lib.W_INT4, _lib.W_FP8])
def test_blocked_layout_addresses(fmt):
    """block_matrix puts every stored byte at the address include/yvmoe.h documents, and
    unblock_matrix inverts it (also on a stacked [X][out][in] tensor)."""
    g = torch.Generator().manual_seed(fmt)
    out, cols = 48, 192                       # 3 row blocks, 3 column blocks
    nbytes = {_lib.W_BF16: cols * 2, _lib.W_INT4: cols // 2}.get(fmt, cols)
    raw = torch.randint(0, 256, (out, nbytes), generator=g, dtype=torch.uint8)
    dt = {_lib.W_BF16: torch.bfloat16, _lib.W_INT8: torch.int8}.get(fmt, torch.uint8)
    q = raw.view(dt)
    b = quant.block_matrix(q, fmt)
    assert b.shape == q.shape and b.dtype == q.dtype
    ub = b.contiguous().view(torch.uint8).flatten()
    for n in range(out):
        for byte in range(nbytes):
            ob, r = divmod(n, 16)
            if fmt == _lib.W_BF16:
                col, half = divmod(byte, 2)
                kb, kk = divmod(col, 64)
                gg, c = divmod(kk, 16)
                h, j = divmod(c, 8)
                off = (ob * (cols // 64) + kb) * 2048 + h * 1024 + (16 * gg + r) * 16 + 2 * j + half
            else:
                piece = 8 if fmt == _lib.W_INT4 else 16
                kb, kk = divmod(byte, 4 * piece)
                gg, c = divmod(kk, piece)
                off = (ob * (cols // 64) + kb) * 64 * piece + (16 * gg + r) * piece + c
            assert int(ub[off]) == int(raw[n, byte])
    assert torch.equal(quant.unblock_matrix(b, fmt).view(torch.uint8), raw)
    st = torch.stack([q, q.flip(0)])
    bs = quant.block_matrix(st, fmt)
    assert torch.equal(bs[0].view(torch.uint8), b.view(torch.uint8))
    assert torch.equal(quant.unblock_matrix(bs, fmt).view(torch.uint8), st.view(torch.uint8))
    f = torch.randn(16, 64, generator=g)
    assert quant.block_matrix(f, _lib.W_F32) is f          # fp32 stays row-major


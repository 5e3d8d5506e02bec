"""Weight formats of the expert FFN and their packers.

Formats (one expert weight is an nn.Linear.weight, [out][in] row-major):

* int8, symmetric per output channel (W8A16):
  ``s = max(amax_row / 127, 1e-8)`` stored as bf16, ``q = clamp(round(w / s), -128, 127)``,
  ``w ~= q * s``. Same arithmetic as ``YvQuantizer.quantize_tensor(bits=8, symmetric=True)``
  (model/utils/quantization.py:337-355) but per output channel, as the W8A16 layer defines.
* int4, group 128 along ``in``, zero point 8 (W4A16): ``s = max(amax_group / 7, 1e-8)``
  stored as bf16 ``[out][in/128]``, ``q = clamp(round(w / s) + 8, 0, 15)``,
  ``w ~= (q - 8) * s``; two codes per byte with the even ``in`` index in the low nibble
  (the convention of opss/optim/ink/kv_cache.py:245, :291-292). The block scheme follows
  ``quantize_to_int4_blockwise`` (opss/quantize/engine.py:889-941) with the zero point
  fixed at 8.
* fp8 e4m3fn (OCP) with 128x128 block scales: ``s = max(amax_block / 448, 1e-12)`` fp32
  ``[out/128][in/128]``, ``q = e4m3fn(clamp(w / s, -448, 448))``, ``w ~= q * s``
  (``quantize_to_fp8`` opss/quantize/engine.py:841-883 with a block granularity, E4M3_MAX
  = 448 at :817).

These run once at weight-load time (torch on whatever device holds the weights); the
forward consumes the packed tensors directly.

Packed layout of the expert matrices (bf16, int8, int4 and fp8; fp32 stays row-major):
16-row x 64-column blocks, each contiguous, blocks ordered row-block major then K. Inside a
block, piece (g, r) = row r (0..15) and columns 16 g .. 16 g + 15 (g = 0..3) sits at
(16 g + r) x piece bytes (16 for 1-byte codes, 8 for int4); bf16 blocks hold the first 8
columns of every piece in their first 1 KB and the last 8 in the second. A wavefront lane
l = 16 g + r of the GEMM kernels needs exactly piece (g, r) of each block, so every weight
load of a 16-column group is one contiguous 1 KB (512 B for int4) read
(:func:`block_matrix`, :func:`unblock_matrix`).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Sequence, Tuple

import torch

from . import _lib

FORMAT_NAMES = {
    _lib.W_F32: "f32",
    _lib.W_BF16: "bf16",
    _lib.W_INT8: "int8",
    _lib.W_INT4: "int4",
    _lib.W_FP8: "fp8",
}
FORMAT_BY_NAME = {v: k for k, v in FORMAT_NAMES.items()}


# ------------------------------------------------------------------ int8
def quantize_int8(w: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    w = w.float()
    s = (w.abs().amax(dim=1) / 127.0).clamp(min=1e-8).to(torch.bfloat16)
    q = torch.round(w / s.float()[:, None]).clamp(-128, 127).to(torch.int8)
    return q, s


def dequantize_int8(q: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    return q.float() * s.float()[:, None]


# ------------------------------------------------------------------ int4 g128
# The kernels' int4 conversion forms (q - 8) * s as (1024 + q) * s - 1032 * s in one fused
# multiply-add, exact (bit-identical to converting q - 8 and multiplying) for bf16 scales with
# 2^-126 <= |s| < 2^97 (and s = 0): above that 1032 * s overflows, below it s / 16 loses bits.
INT4_SCALE_MIN, INT4_SCALE_MAX = 2.0 ** -126, 2.0 ** 97


def check_int4_scales(s: torch.Tensor, what: str = "int4 scales") -> None:
    """Raise ValueError for a bf16 group scale the kernels cannot apply exactly: not finite,
    |s| >= 2^97, or 0 < |s| < 2^-126 (subnormal)."""
    a = s.float().abs()
    bad = ~torch.isfinite(a) | (a >= INT4_SCALE_MAX) | ((a > 0) & (a < INT4_SCALE_MIN))
    if bool(bad.any()):
        v = float(s.float().reshape(-1)[bad.reshape(-1)][0])
        raise ValueError(f"{what}: scale {v!r} outside the supported range 2^-126 <= |s| < 2^97 "
                         f"(or 0)")


def quantize_int4(w: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    w = w.float()
    out, inn = w.shape
    if inn % 128:
        raise ValueError(f"int4 group-128 needs in % 128 == 0, got {inn}")
    wg = w.view(out, inn // 128, 128)
    s = (wg.abs().amax(dim=-1) / 7.0).clamp(min=1e-8).to(torch.bfloat16)
    check_int4_scales(s, "int4 quantization")
    q = (torch.round(wg / s.float()[..., None]) + 8).clamp(0, 15).to(torch.uint8).view(out, inn)
    packed = q[:, 0::2] | (q[:, 1::2] << 4)
    return packed.contiguous(), s


def unpack_int4(packed: torch.Tensor) -> torch.Tensor:
    lo = packed & 0xF
    hi = packed >> 4
    return torch.stack([lo, hi], dim=-1).view(packed.shape[0], packed.shape[1] * 2)


def dequantize_int4(packed: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    q = unpack_int4(packed).float() - 8.0
    out, inn = q.shape
    return (q.view(out, inn // 128, 128) * s.float()[..., None]).view(out, inn)


# ------------------------------------------------------------------ fp8 e4m3fn, 128x128 blocks
E4M3_MAX = 448.0


def quantize_fp8(w: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    w = w.float()
    out, inn = w.shape
    if out % 128 or inn % 128:
        raise ValueError(f"fp8 128x128 blocks need out, in % 128 == 0, got {tuple(w.shape)}")
    wb = w.view(out // 128, 128, inn // 128, 128)
    s = (wb.abs().amax(dim=(1, 3)) / E4M3_MAX).clamp(min=1e-12)
    q = (wb / s[:, None, :, None]).clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)
    return q.view(out, inn).view(torch.uint8).contiguous(), s.contiguous()


def dequantize_fp8(q: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    out, inn = q.shape
    v = q.view(torch.float8_e4m3fn).float().view(out // 128, 128, inn // 128, 128)
    return (v * s.float()[:, None, :, None]).view(out, inn)


# ------------------------------------------------------------------ blocked layout
BLOCKED_FORMATS = (_lib.W_BF16, _lib.W_INT8, _lib.W_INT4, _lib.W_FP8)


def _block_view(t: torch.Tensor, fmt: int):
    """[..., out, row_bytes] (uint8 view) -> the 6-/7-d view whose permutation is the layout."""
    *lead, out, nb = t.shape
    if fmt == _lib.W_BF16:       # 64 columns = 128 B per row-block row: [kb][g][h][16 B]
        return t.reshape(*lead, out // 16, 16, nb // 128, 4, 2, 16)
    piece = 8 if fmt == _lib.W_INT4 else 16
    return t.reshape(*lead, out // 16, 16, nb // (4 * piece), 4, piece)


def block_matrix(q: torch.Tensor, fmt: int) -> torch.Tensor:
    """Stored codes [..., out, in-bytes] in row-major order -> the blocked layout (same shape
    and dtype, elements reordered). out % 16 == 0 and in % 64 == 0 are required."""
    if fmt not in BLOCKED_FORMATS:
        return q
    u = q.contiguous().view(torch.uint8)
    v = _block_view(u, fmt)
    n = v.dim()
    if fmt == _lib.W_BF16:       # (..., ob, r, kb, g, h, b) -> (..., ob, kb, h, g, r, b)
        o = list(range(n - 6)) + [n - 6, n - 4, n - 2, n - 3, n - 5, n - 1]
    else:                        # (..., ob, r, kb, g, b) -> (..., ob, kb, g, r, b)
        o = list(range(n - 5)) + [n - 5, n - 3, n - 2, n - 4, n - 1]
    return v.permute(*o).contiguous().view(u.shape).view(q.dtype)


def unblock_matrix(b: torch.Tensor, fmt: int) -> torch.Tensor:
    """Inverse of :func:`block_matrix`."""
    if fmt not in BLOCKED_FORMATS:
        return b
    u = b.contiguous().view(torch.uint8)
    *lead, out, nb = u.shape
    if fmt == _lib.W_BF16:
        v = u.reshape(*lead, out // 16, nb // 128, 2, 4, 16, 16)     # (ob, kb, h, g, r, b)
        n = v.dim()
        o = list(range(n - 6)) + [n - 6, n - 2, n - 5, n - 3, n - 4, n - 1]
    else:
        piece = 8 if fmt == _lib.W_INT4 else 16
        v = u.reshape(*lead, out // 16, nb // (4 * piece), 4, 16, piece)  # (ob, kb, g, r, b)
        n = v.dim()
        o = list(range(n - 5)) + [n - 5, n - 2, n - 4, n - 3, n - 1]
    return v.permute(*o).contiguous().view(u.shape).view(b.dtype)


# ------------------------------------------------------------------ packed expert stack
@dataclass
class PackedExperts:
    """Routed experts [0, E) and shared experts [E, E+S) stacked in one format.

    w_gate/w_up [E+S][F][H], w_down [E+S][H][F] (int4: last dim halved, uint8) in the
    blocked layout of :func:`block_matrix` (fp32: row-major), scales row-major as documented
    in include/yvmoe.h.
    """

    format: int
    num_routed: int
    num_shared: int
    hidden: int
    ffn: int
    w_gate: torch.Tensor
    w_up: torch.Tensor
    w_down: torch.Tensor
    s_gate: Optional[torch.Tensor] = None
    s_up: Optional[torch.Tensor] = None
    s_down: Optional[torch.Tensor] = None

    @property
    def num_total(self) -> int:
        return self.num_routed + self.num_shared

    def tensors(self):
        return [t for t in (self.w_gate, self.w_up, self.w_down, self.s_gate, self.s_up, self.s_down)
                if t is not None]

    def to(self, device) -> "PackedExperts":
        f = lambda t: None if t is None else t.to(device)
        return PackedExperts(self.format, self.num_routed, self.num_shared, self.hidden, self.ffn,
                             f(self.w_gate), f(self.w_up), f(self.w_down), f(self.s_gate),
                             f(self.s_up), f(self.s_down))

    def struct(self) -> _lib.ExpertWeights:
        p = lambda t: None if t is None else t.data_ptr()
        return _lib.ExpertWeights(self.format, self.num_routed, self.num_shared, self.hidden,
                                  self.ffn, p(self.w_gate), p(self.w_up), p(self.w_down),
                                  p(self.s_gate), p(self.s_up), p(self.s_down))

    def weight_bytes(self, expert: int) -> int:
        """Bytes of one expert's three matrices and their scales."""
        return sum(t[expert].numel() * t.element_size() for t in self.tensors())

    def dequantize(self, expert: int, dtype=torch.float32):
        """(Wg, Wu, Wd) of one expert as dense [out][in] tensors (for checkers)."""
        fmt = self.format
        res = []
        for w, s in ((self.w_gate, self.s_gate), (self.w_up, self.s_up), (self.w_down, self.s_down)):
            we = unblock_matrix(w[expert], fmt)
            if fmt in (_lib.W_F32, _lib.W_BF16):
                d = we.float()
            elif fmt == _lib.W_INT8:
                d = dequantize_int8(we, s[expert])
            elif fmt == _lib.W_INT4:
                d = dequantize_int4(we, s[expert])
            else:
                d = dequantize_fp8(we, s[expert])
            res.append(d.to(dtype))
        return tuple(res)


def quantize_matrix(w: torch.Tensor, fmt: int):
    """One [out][in] matrix -> (stored tensor, scale or None)."""
    if fmt == _lib.W_F32:
        return w.float().contiguous(), None
    if fmt == _lib.W_BF16:
        return w.to(torch.bfloat16).contiguous(), None
    if fmt == _lib.W_INT8:
        return quantize_int8(w)
    if fmt == _lib.W_INT4:
        return quantize_int4(w)
    if fmt == _lib.W_FP8:
        return quantize_fp8(w)
    raise ValueError(f"unknown weight format {fmt}")


class ExpertPacker:
    """Fills a PackedExperts one expert at a time (bounded memory for large layers)."""

    def __init__(self, fmt: int, num_routed: int, num_shared: int, hidden: int, ffn: int, device):
        self.fmt = fmt
        self.E, self.S, self.H, self.F = num_routed, num_shared, hidden, ffn
        X = num_routed + num_shared
        H, F = hidden, ffn
        dev = torch.device(device)
        if fmt == _lib.W_F32:
            mk = lambda o, i: torch.empty(X, o, i, dtype=torch.float32, device=dev)
            sk = lambda o, i: None
        elif fmt == _lib.W_BF16:
            mk = lambda o, i: torch.empty(X, o, i, dtype=torch.bfloat16, device=dev)
            sk = lambda o, i: None
        elif fmt == _lib.W_INT8:
            mk = lambda o, i: torch.empty(X, o, i, dtype=torch.int8, device=dev)
            sk = lambda o, i: torch.empty(X, o, dtype=torch.bfloat16, device=dev)
        elif fmt == _lib.W_INT4:
            mk = lambda o, i: torch.empty(X, o, i // 2, dtype=torch.uint8, device=dev)
            sk = lambda o, i: torch.empty(X, o, i // 128, dtype=torch.bfloat16, device=dev)
        elif fmt == _lib.W_FP8:
            mk = lambda o, i: torch.empty(X, o, i, dtype=torch.uint8, device=dev)
            sk = lambda o, i: torch.empty(X, o // 128, i // 128, dtype=torch.float32, device=dev)
        else:
            raise ValueError(f"unknown weight format {fmt}")
        self.packed = PackedExperts(fmt, num_routed, num_shared, H, F, mk(F, H), mk(F, H), mk(H, F),
                                    sk(F, H), sk(F, H), sk(H, F))

    def set(self, expert: int, wg: torch.Tensor, wu: torch.Tensor, wd: torch.Tensor) -> None:
        p = self.packed
        for w, dst, sdst in ((wg, p.w_gate, p.s_gate), (wu, p.w_up, p.s_up), (wd, p.w_down, p.s_down)):
            q, s = quantize_matrix(w.to(dst.device), self.fmt)
            dst[expert].copy_(block_matrix(q, self.fmt))
            if sdst is not None:
                sdst[expert].copy_(s)


def pack_experts(weights: Sequence[Tuple[torch.Tensor, torch.Tensor, torch.Tensor]], num_routed: int,
                 fmt: int, device=None) -> PackedExperts:
    """Pack a list of (Wg [F,H], Wu [F,H], Wd [H,F]) (routed first, then shared)."""
    F, H = weights[0][0].shape
    dev = device if device is not None else weights[0][0].device
    pk = ExpertPacker(fmt, num_routed, len(weights) - num_routed, H, F, dev)
    for i, (wg, wu, wd) in enumerate(weights):
        pk.set(i, wg, wu, wd)
    return pk.packed


# ------------------------------------------------------------------ router
def split_bf16x3(w: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """fp32 w -> (hi, mid, lo) bf16 with hi + mid + lo == w to within one fp32 ulp."""
    w = w.float()
    hi = w.to(torch.bfloat16)
    r1 = w - hi.float()
    mid = r1.to(torch.bfloat16)
    r2 = r1 - mid.float()
    lo = r2.to(torch.bfloat16)
    return hi, mid, lo


def pack_router(gate_weight: torch.Tensor, pred_w1: Optional[torch.Tensor], act: int) -> torch.Tensor:
    """Router GEMM operand: [gate.weight padded to Ep rows; predictor W1 terms] ([out][H]).

    bf16 activations: bf16 [Ep + 192][H] with W1 split into three bf16 terms so the bf16
    MFMA reproduces the fp32 predictor (complexity_predictor is fp32, gate.py:930-936), in
    the blocked order of :func:`block_matrix`. fp32 activations: fp32 [Ep + 64][H] row-major.
    """
    E, H = gate_weight.shape
    Ep = (E + 15) // 16 * 16
    dev = gate_weight.device
    if pred_w1 is None:
        pred_w1 = torch.zeros(_lib.PREDICTOR_DIM, H, device=dev)
    if act == _lib.ACT_BF16:
        g = torch.zeros(Ep, H, dtype=torch.bfloat16, device=dev)
        g[:E] = gate_weight.to(torch.bfloat16)
        hi, mid, lo = split_bf16x3(pred_w1.to(dev))
        return block_matrix(torch.cat([g, hi, mid, lo], dim=0).contiguous(), _lib.W_BF16)
    g = torch.zeros(Ep, H, dtype=torch.float32, device=dev)
    g[:E] = gate_weight.float()
    return torch.cat([g, pred_w1.float().to(dev)], dim=0).contiguous()

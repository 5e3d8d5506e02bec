"""Shared test helpers: oracle parameters of a workload, comparison metrics, and the parity
record every GPU comparison adds to (printed as the "parity summary" at the end of a pytest
run, including under -q, by tests/conftest.py)."""
import torch

from oracle.moe_oracle import params_from_workload as oracle_params  # noqa: F401

BF16_MAX_ABS, BF16_COS = 2e-2, 0.9999
F32_MAX_ABS, F32_COS = 1e-4, 0.999999

# one entry per comparison: (label, elements, max_abs, cosine, elements above the max-abs
# bound, dtype)
PARITY_RECORDS = []


def cosine(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.double().reshape(-1)
    b = b.double().reshape(-1)
    return float((a @ b) / (a.norm() * b.norm() + 1e-300))


def max_abs(a: torch.Tensor, b: torch.Tensor) -> float:
    return float((a.double() - b.double()).abs().max())


def bf16_ulp(v: torch.Tensor) -> torch.Tensor:
    """Spacing of bf16 numbers at |v| (2^(floor(log2|v|) - 7))."""
    a = v.double().abs().clamp(min=2.0 ** -126)
    return torch.exp2(torch.floor(torch.log2(a)) - 7)


def bf16_allowance(want: torch.Tensor) -> torch.Tensor:
    """Per-element bound of the bf16 layer-output check: 2e-2, widened only where |want| >= 2,
    to two bf16 steps in [2, 4) (0.03125; the reference's own bf16 chain, torch's F.linear,
    lands two steps from the correctly rounded value there at cfg4, pinned by
    tests/test_oracle_bf16_envelope.py) and to one step, i.e. the adjacent bf16 value, from 4 up
    (the least by which two roundings of nearly the same fp32 sum can differ)."""
    a = want.double().abs()
    ulp = bf16_ulp(want)
    steps = torch.where(a < 4.0, torch.full_like(a, 2.0), torch.ones_like(a))
    wide = torch.where(a >= 2.0, steps * ulp, torch.zeros_like(a))
    return torch.maximum(torch.full_like(a, BF16_MAX_ABS), wide)


def check_close(got: torch.Tensor, want: torch.Tensor, label: str):
    """Layer-output tolerance. fp32: max-abs <= 1e-4 and cosine >= 0.999999. bf16: cosine >=
    0.9999 and every element within ``bf16_allowance`` of the reference value (2e-2; at |want|
    in [2, 4) two bf16 steps = 0.03125, from 4 up the adjacent bf16 value), with at most 1e-5
    of the elements beyond 2e-2. Records the comparison for the parity summary; returns
    (max_abs, cosine, elements above 2e-2)."""
    got, want = got.cpu(), want.cpu()
    if want.dtype == torch.float32:
        tol_abs, tol_cos = F32_MAX_ABS, F32_COS
    else:
        tol_abs, tol_cos = BF16_MAX_ABS, BF16_COS
    d = (got.double() - want.double()).abs()
    if want.dtype == torch.bfloat16:
        bound = bf16_allowance(want)
    else:
        bound = torch.full_like(d, tol_abs)
    beyond = int((d > bound).sum()) if d.numel() else 0
    over = int((d > tol_abs).sum()) if d.numel() else 0
    ma = float(d.max()) if d.numel() else 0.0
    cs = cosine(got, want) if d.numel() else 1.0
    PARITY_RECORDS.append((label, d.numel(), ma, cs, over, str(want.dtype).replace("torch.", "")))
    print(f"parity {label}: max_abs={ma:.3e} cos={cs:.7f} above_{tol_abs:g}={over}/{d.numel()}",
          flush=True)
    assert beyond == 0, f"{label}: {beyond} elements beyond the bf16 allowance; max_abs={ma}"
    assert over <= 1e-5 * d.numel(), f"{label}: {over} elements above {tol_abs}; max_abs={ma}"
    assert cs >= tol_cos, f"{label}: cosine {cs}"
    return ma, cs, over


def check_ulps(got: torch.Tensor, want: torch.Tensor, label: str, max_ulps: int = 2):
    """Intermediate bf16 GEMM outputs (expert rows [R, H]) against the oracle's correctly
    rounded values: every element within ``max_ulps`` bf16 ulps, measured at the larger of
    its two magnitudes and the rms of its row (an fp32 sum in another order, rounded once,
    lands on the same or a neighbouring bf16 value; a one-ulp step in an input element, the
    bf16 intermediate h, moves the sum by an amount set by the row's scale, not by the
    element's own size, which can be near zero after cancellation), cosine >= 0.99999.
    Recorded for the parity summary with the count of elements that differ."""
    got, want = got.cpu().double(), want.cpu().double()
    d = (got - want).abs()
    rms = want.pow(2).mean(dim=-1, keepdim=True).sqrt().expand_as(want)
    ulp = torch.maximum(torch.maximum(bf16_ulp(got), bf16_ulp(want)), bf16_ulp(rms))
    n_ulps = float((d / ulp).max()) if d.numel() else 0.0
    differ = int((d > 0).sum())
    ma = float(d.max()) if d.numel() else 0.0
    cs = cosine(got, want) if d.numel() else 1.0
    PARITY_RECORDS.append((label, d.numel(), ma, cs, differ, "bf16-ulp"))
    print(f"parity {label}: max_abs={ma:.3e} max_ulps={n_ulps:.2f} cos={cs:.7f} "
          f"differ={differ}/{d.numel()}", flush=True)
    assert n_ulps <= max_ulps, f"{label}: {n_ulps} ulps"
    assert cs >= 0.99999, f"{label}: cosine {cs}"

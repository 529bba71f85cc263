"""Error bounds shared by the GPU parity tests.

A kernel that accumulates in fp32 and rounds its result once to the output
dtype may differ from the float64 oracle by its own arithmetic error (the
absolute term of each bound) plus that final rounding: half an ulp of the
result.  Relative to |ref| the half-ulp lies between 2^-(p+1) and 2^-p for a
p-bit significand (bf16: p = 8, so 2^-9 .. 2^-8), so the rounding term is
computed per element from the exponent of the reference value instead of
being folded into one relative factor.
"""
import torch

_MANTISSA = {torch.bfloat16: 7, torch.float16: 10, torch.float32: 23}


def half_ulp(ref, dtype):
    """Half an ulp of each element of ``ref`` in ``dtype`` (0 where ref is 0)."""
    ref = ref.double()
    _, e = torch.frexp(ref)                     # |ref| = m * 2^e, m in [0.5, 1)
    ulp = torch.ldexp(torch.ones_like(ref), (e - 1 - _MANTISSA[dtype]).to(torch.int64))
    return torch.where(ref == 0, torch.zeros_like(ref), ulp / 2)


def excess(actual, expected, atol, out_dtype, rtol=0.0):
    """max(|actual - expected| - (atol + rtol*|ref| + half_ulp(ref))) and max |error|."""
    a = actual.detach().cpu().double()
    e = expected.detach().cpu().double()
    assert torch.isfinite(a).all(), 'non-finite output'
    err = (a - e).abs()
    bound = atol + rtol * e.abs() + half_ulp(e, out_dtype)
    return (err - bound).max().item(), err.max().item()

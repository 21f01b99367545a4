"""Relative tolerance policy (reference `tests/tolerance.py:35-170`).

truth = the fp64 oracle with the selection computed once from the
low-precision inputs and held fixed; ref_error = the same oracle evaluated
in the target dtype. A result passes when its max-abs error against truth is
within max(TOLERANCE_FACTOR * ref_error, TOLERANCE_FLOOR). Selection is
compared exactly, never within a tolerance.

Also the absolute bars BASELINE's north star states for bf16 (max-abs <=
2e-2, mean-abs <= 2e-3) and for the float32 path (max-abs <= 1e-5).
"""

import torch

from oracle import naive as O

TOLERANCE_FACTOR = 2.0
TOLERANCE_FLOOR = 1e-6
BF16_MAX_ABS = 2e-2
BF16_MEAN_ABS = 2e-3
FP32_MAX_ABS = 1e-5


def max_abs_error(a, b) -> float:
    return (a.double().cpu() - b.double().cpu()).abs().max().item()


def mean_abs_error(a, b) -> float:
    return (a.double().cpu() - b.double().cpu()).abs().mean().item()


def assert_selection_matches(actual, expected, name):
    if actual.shape != expected.shape:
        raise AssertionError(f"{name}: selection shape {tuple(actual.shape)} != "
                             f"oracle {tuple(expected.shape)}")
    bad = (actual.cpu() != expected.cpu())
    if bool(bad.any()):
        per_q = bad.any(dim=-1)
        first = torch.nonzero(per_q)[0].tolist()
        raise AssertionError(
            f"{name}: block selection differs from oracle for {int(per_q.sum())}/"
            f"{per_q.numel()} queries; first at [b,h,s]={first}. This is a routing bug, "
            f"not a precision issue.")


def assert_within_tolerance(actual, truth, ref_error, name):
    budget = max(TOLERANCE_FACTOR * ref_error, TOLERANCE_FLOOR)
    err = max_abs_error(actual, truth)
    if err > budget:
        raise AssertionError(f"{name}: max abs error {err:.3e} exceeds tolerance "
                             f"{budget:.3e} (reference error {ref_error:.3e} x "
                             f"{TOLERANCE_FACTOR})")

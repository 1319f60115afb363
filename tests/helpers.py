"""Shared helpers for the parity tests (comparison rules and tensor glue)."""
from __future__ import annotations

import numpy as np

# North-star parity bar on bf16 outputs.
MAX_ABS = 2e-2
MEAN_ABS = 2e-3


def bf16_bits_to_f32(h) -> np.ndarray:
    return (np.ascontiguousarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def nearly_equal_mask(got, exp, atol, rtol):
    """The reference's comparison rule, tests/test_helpers.h:70-72:
    |a - b| <= atol + rtol * |b|."""
    return np.abs(got - exp) <= atol + rtol * np.abs(exp)


def check_close(got, exp, atol, rtol, label=""):
    got = np.asarray(got, np.float32)
    exp = np.asarray(exp, np.float32)
    assert got.shape == exp.shape, f"{label}: shape {got.shape} != {exp.shape}"
    ok = nearly_equal_mask(got, exp, atol, rtol)
    if not ok.all():
        idx = np.flatnonzero(~ok.reshape(-1))[0]
        raise AssertionError(
            f"{label}: {int((~ok).sum())} mismatches, first at flat {idx}: "
            f"expected {exp.reshape(-1)[idx]!r}, got {got.reshape(-1)[idx]!r}")


def parity_stats(got, exp):
    d = np.abs(np.asarray(got, np.float64) - np.asarray(exp, np.float64))
    return float(d.max()) if d.size else 0.0, float(d.mean()) if d.size else 0.0


def check_bar(got, exp, label="", max_abs=MAX_ABS, mean_abs=MEAN_ABS):
    """max-abs <= 2e-2 and mean-abs <= 2e-3 on bf16 outputs."""
    assert np.isfinite(got).all(), f"{label}: non-finite output"
    mx, mn = parity_stats(got, exp)
    assert mx <= max_abs and mn <= mean_abs, f"{label}: max-abs {mx:.3g}, mean-abs {mn:.3g}"
    return mx, mn


# --------------------------------------------------------- torch glue (GPU)

def to_dev_bf16(bits: np.ndarray, dev):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(bits, dtype=np.uint16).view(np.int16))
    return t.view(torch.bfloat16).to(dev)


def from_dev_bf16(t) -> np.ndarray:
    import torch

    return t.detach().to("cpu").contiguous().view(torch.int16).numpy().view(np.uint16)


def to_dev_f32(a: np.ndarray, dev):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)


def sync():
    import torch

    torch.cuda.synchronize()

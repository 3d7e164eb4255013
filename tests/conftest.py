from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU and the built HIP library")


def golden(name: str) -> dict[str, np.ndarray]:
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as data:
        return {key: data[key] for key in data.files}


def bf16_parity(tag: str, got, want16, want32, *, slack: float = 1.25,
                max_slack: float | None = None, min_inside: float = 0.985, rtol: float = 2e-2,
                atol: float = 2e-2, elementwise: bool = True) -> None:
    """The 16-bit parity bar, for results the reference's own 16-bit path cannot itself
    reproduce to an elementwise 2e-2 of FP32.

    ``got`` is the HIP result in 16 bits, ``want16`` the oracle run in the same 16-bit mode
    (the reference's portable path) and ``want32`` the oracle in FP32 on the same inputs and
    16-bit-valued weights. Asserts that the HIP result is at least as accurate as the
    reference's 16-bit path, within ``slack`` (``max_slack`` for the max error, default
    ``slack``):

    * in norm and in max abs error against the FP32 result;
    * elementwise: it misses the bar ``atol + rtol |x|`` of the FP32 result on at most
      ``slack`` times as many elements as the reference's 16-bit path does, plus the counting
      noise of a small count (4 sqrt(count) + 8: 6 reference misses allow 25, 166k allow 209k);

    and, with ``elementwise`` (single passes, where two 16-bit paths stay close), that it
    agrees with the reference's 16-bit result to the same bar on at least ``min_inside`` of the
    elements, with no element further from it than the reference's own largest 16-bit error
    plus the bar. Callers set ``min_inside`` a little below the fraction the HIP path reaches on
    their inputs (the default, 98.5%, covers the small random-input scans, which reach 98.8% and
    more); a regression that doubles the disagreement then fails. (Long 16-bit chains such as a
    24-layer decode drift from FP32 and from each other by more than the bar; there only the
    accuracy checks apply.)
    """
    import torch

    got, want16, want32 = got.float().cpu(), want16.float().cpu(), want32.float().cpu()
    e_got = (got - want32).abs()
    e_ref = (want16 - want32).abs()
    bar32 = atol + rtol * want32.abs()
    out_got, out_ref = int((e_got > bar32).sum()), int((e_ref > bar32).sum())
    d = (got - want16).abs()
    inside = (d <= atol + rtol * want16.abs()).float().mean().item()
    n_got, n_ref = e_got.norm().item(), e_ref.norm().item()
    m_got, m_ref = e_got.max().item(), e_ref.max().item()
    print(f"{tag}: vs FP32 ||e|| {n_got:.3e} (reference 16-bit {n_ref:.3e}), max {m_got:.3e} "
          f"(reference {m_ref:.3e}), outside the bar {out_got} (reference {out_ref}) of "
          f"{got.numel()}; vs reference 16-bit: max {d.max().item():.3e}, "
          f"{100 * (1 - inside):.3f}% outside {atol:.0e} + {rtol:.0e}|x|", flush=True)
    assert n_got <= slack * n_ref + 1e-30, f"{tag}: norm error {n_got:.3e} > {slack} x {n_ref:.3e}"
    ms = slack if max_slack is None else max_slack
    assert m_got <= ms * m_ref + 1e-30, f"{tag}: max error {m_got:.3e} > {ms} x {m_ref:.3e}"
    assert out_got <= slack * out_ref + 4.0 * out_ref ** 0.5 + 8, (
        f"{tag}: {out_got} elements outside the bar of FP32, the reference {out_ref}")
    if elementwise:
        assert inside >= min_inside, f"{tag}: only {inside:.4f} of elements within the bar"
        assert bool((d <= m_ref + atol + rtol * want16.abs()).all()), f"{tag}: an outlier"

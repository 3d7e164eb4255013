"""Host-side checks of the scalar math the kernels share (``mamba3_amd/csrc/m3_math.h``)."""

from __future__ import annotations

import os
import shutil
import subprocess

import numpy as np
import pytest

from conftest import ROOT

HEADER_DIR = os.path.join(ROOT, "mamba3_amd", "csrc")

PROGRAM = r"""
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include "m3_math.h"
int main(int argc, char** argv) {
  /* read float32 values from stdin (binary), write fmodf and m3_fmod_2pi results */
  float x;
  while (fread(&x, sizeof x, 1, stdin) == 1) {
    float a = fmodf(x, M3_TWO_PI_F), b = m3_fmod_2pi(x);
    fwrite(&a, sizeof a, 1, stdout);
    fwrite(&b, sizeof b, 1, stdout);
  }
  return 0;
}
"""


@pytest.fixture(scope="module")
def fmod_bin(tmp_path_factory):
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    d = tmp_path_factory.mktemp("m3math")
    src, exe = d / "t.c", d / "t"
    src.write_text(PROGRAM)
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", f"-I{HEADER_DIR}", str(src), "-o",
                    str(exe), "-lm"], check=True)
    return str(exe)


def _run(exe, x: np.ndarray):
    out = subprocess.run([exe], input=x.astype(np.float32).tobytes(), capture_output=True,
                         check=True).stdout
    pairs = np.frombuffer(out, dtype=np.float32).reshape(-1, 2)
    return pairs[:, 0], pairs[:, 1]


def test_fast_fmod_equals_fmodf(fmod_bin):
    rng = np.random.default_rng(0)
    c = np.float32(6.28318530717958647692)
    parts = [
        rng.uniform(-1e4, 1e4, 200_000),
        rng.uniform(-500, 500, 200_000),
        rng.uniform(-7, 7, 200_000),
        rng.standard_normal(100_000) * 1e-3,
        # values within a few ulps of multiples of 2 pi, where the quotient can be off by one
        (np.arange(-3000, 3000)[:, None] * c + np.linspace(-3e-3, 3e-3, 41)[None, :]).ravel(),
        np.nextafter(np.arange(-2000, 2000) * c, np.inf),
        np.nextafter(np.arange(-2000, 2000) * c, -np.inf),
        np.array([0.0, -0.0, c, -c, 2 * c, 1e7, -1e7, 3e9], dtype=np.float32),
    ]
    x = np.concatenate([p.astype(np.float32) for p in parts])
    want, got = _run(fmod_bin, x)
    np.testing.assert_array_equal(got, want)

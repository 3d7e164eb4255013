"""The bench's roofline accounting against the per-config figures it is quoted with.

Algorithmic bytes and FLOPs are closed forms of the configuration: config 2 prefill reads the
in_proj output once and writes y once (13,056 B per token), and its chunked SSD at the
reference chunk (256) needs 82,112 FLOP per (token, head); a decode step streams the FP32 state
once each way plus the per-row vectors (4,277,568 B per layer and row at rank 1, 4,377,408 at
rank 4). The committed counter summaries must parse to the HBM bytes the JSON line reports.
"""

from __future__ import annotations

import os

import bench


def test_prefill_bytes_and_flops_of_config_2():
    proj = 2 * 2048 + 2 * 128 + 3 * 32 + 32  # z, x, B, C, dt, A, trap, angles
    assert proj == 4480
    assert bench.prefill_bytes(8, 8192, 1024, proj) == 855_638_016
    assert bench.prefill_bytes(8, 8192, 1024, proj) // (8 * 8192) == 13_056
    flops = bench.prefill_flops(8, 8192, 32, 128, 64, 1, 256)
    assert flops == 8 * 8192 * 32 * 82_112 == 172_201_345_024


def test_prefill_flops_of_config_3_per_layer():
    assert bench.prefill_flops(8, 4096, 32, 128, 64, 4, 32) == 8 * 4096 * 32 * 232_448


def test_decode_bytes_per_layer_row():
    assert bench.decode_bytes_per_layer_row(64, 64, 128, 32, 1) == 4_277_568
    assert bench.decode_bytes_per_layer_row(64, 64, 128, 32, 4) == 4_377_408


def test_committed_counter_summaries_parse():
    scan = bench._traffic_from_profile(os.path.join(bench.ROOT, "profiles", "scan_config2_pmc.txt"))
    step = bench._traffic_from_profile(
        os.path.join(bench.ROOT, "profiles", "step_decode_b256_pmc.txt"),
        key="traffic_bytes_per_launch:")
    assert scan is not None and 855_638_016 < scan < 2 * 855_638_016
    assert step is not None and 1_095_057_408 <= step < 1.1 * 1_095_057_408

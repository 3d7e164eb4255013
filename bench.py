"""Benchmark of the Mamba-3 mixer hot path on one MI355X.

Headline workload: the SISO prefill scan of
``Mamba3(d_model=1024, d_state=128, depth=1, mimo_rank=1)`` on ``x [8, 8192, 1024]`` under
bf16 autocast, seed 1. A step is one ``m3_scan_fwd`` call (its prep kernel: the RMS-normalized
B/C rows, pi tanh(angle), the per-(head, sub-chunk) dt / A / trapezoid scalars; then the
16-wave scan kernel: bounded phase, bias, rotation, chunked SSD, D skip, SiLU gate) over the
whole batch, with its input, the ``in_proj`` output, already resident in HBM, timed with HIP
events on the launch stream. The timed calls follow the forward line's 30 passes, which run
the same kernels, so they are timed at the GPU's sustained-load clock. ``value`` is prefill
tokens/s of that call. Also reported, in the same JSON line:

* ``roofline``: the call against the HBM roof (its binding roof: arithmetic intensity
  ~201 flop/B at the reference chunk is below the MI355X ridge of ~315 flop/B), ``traffic``
  from the committed PMC summary ``profiles/scan_config2_pmc.txt``;
  ``roofline_mfma``: the same kernel against dense bf16 MFMA;
* ``forward``: tokens/s of the whole mixer forward (norm, in_proj, scan, out_proj, residual);
* ``decode``: BASELINE.json configs[3], ``Mamba3(2048, 128, 24, 1)`` with bf16 weights and an
  FP32 state, 2048-token prefill, then 512 hipGraph replays of ``step`` at B = 256, plus the
  step kernel alone against the HBM roof;
* ``cpu_baseline``: the CPU oracle (a restatement of the reference's portable path) on a
  bounded sample of the same scan, on this host's cores.

Usage: ``python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-decode] [--no-cpu]
[--copy-probe]``.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
MFMA_BF16_PEAK_TFLOPS = 2500.0  # dense bf16 MFMA
METRIC = "prefill tok/s (B=8,L=8K) + decode tok/s (B=256) on 1 GPU; % MFMA/HBM roofline"
FWD_ITERS = 30  # timed config-2 forward passes (run before the headline scan calls)


def prefill_bytes(batch, length, d_model, proj):
    """Algorithmic bytes of one scan launch: the in_proj output read once, y written once."""
    return batch * length * (2 * proj + 2 * 2 * d_model)


def prefill_flops(batch, length, heads, n, p, rank, chunk):
    """Chunked-SSD FLOPs (causal lower triangle incl. diagonal) at chunk size ``chunk``."""
    return batch * length * heads * ((chunk + 1) * rank * rank * (n + p) + 4 * rank * n * p)


def decode_bytes_per_layer_row(heads, p, n, s, rank):
    """Bytes one decode step moves per (layer, batch row) in the step kernel."""
    return (2 * heads * p * n * 4 + heads * (4 * rank * n + 8 * p + 8 * s + 12)
            + 4 * rank * n + 2 * s)


def _events_time(fn, iters):
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(iters):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / 1000.0


def _traffic_from_profile(path, key="traffic_bytes_per_call:"):
    """HBM bytes per call or launch as recorded by a committed PMC summary (or None).

    The summary holds one line ``<key> <int>``: FETCH_SIZE and WRITE_SIZE of the measured
    kernels, each scaled by the counter's reading for a copy of known size.
    """
    try:
        with open(path) as f:
            for line in f:
                if line.startswith(key):
                    return int(line.split(":", 1)[1].strip())
    except OSError:
        return None
    return None


def prepare_prefill():
    """Config 2's model, input and its prepared scan call (the headline workload)."""
    from mamba3_amd import Mamba3, ops

    dev = torch.device("cuda:0")
    torch.manual_seed(1)
    model = Mamba3(1024, d_state=128, depth=1, mimo_rank=1).eval()
    x = torch.randn(8, 8192, 1024)
    model = model.to(dev)
    x = x.to(dev)
    mixer = model.layers[0].mixer
    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.bfloat16):
        proj = mixer.in_proj(model.layers[0].norm(x))
        # one prepared m3_scan_fwd call (prep + scan kernels), relaunched back to back
        call = ops.ScanCall(proj, mixer, chunk_size=mixer.inference_chunk_size)
    torch.cuda.synchronize()
    return dict(model=model, x=x, mixer=mixer, proj=proj, call=call)


def bench_prefill(prep, steps, warmup, log, copy_probe=False):
    from mamba3_amd import ops

    dev = torch.device("cuda:0")
    model, x, mixer, call = prep["model"], prep["x"], prep["mixer"], prep["call"]
    batch, length = x.shape[:2]
    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.bfloat16):
        # The forward line first: its passes run the same scan kernels (and the projection
        # GEMMs) for ~40 ms, so the timed scan calls below find the GPU at the clocks of
        # sustained prefill load. Right after a change of workload the shader clock runs at
        # 1.8-2.2 GHz for the first tens of dispatches before it settles at 2.4 GHz (per-dispatch
        # GRBM_GUI_ACTIVE / duration), and a 5-call warmup alone would time that ramp.
        def forward():
            model(x)

        for _ in range(2):
            forward()
        t_fwd = _events_time(forward, FWD_ITERS)
        for _ in range(warmup):
            call.launch()
        assert ops._HIP_LAST_SCAN_DISPATCH
        t_scan = _events_time(call.launch, steps)
    if copy_probe:
        # a plain 1 GiB device copy: the reference reading for the PMC byte counters
        src_buf = torch.ones(256 * 1024 * 1024, device=dev)
        dst_buf = torch.empty_like(src_buf)
        dst_buf.copy_(src_buf)
        torch.cuda.synchronize()
        del src_buf, dst_buf
    per_launch = t_scan / steps
    tokens = batch * length
    proj_size = mixer.in_proj.weight.shape[0]
    nbytes = prefill_bytes(batch, length, 1024, proj_size)
    flops_ref = prefill_flops(batch, length, mixer.nheads, 128, mixer.headdim, 1, 256)
    flops_own = prefill_flops(batch, length, mixer.nheads, 128, mixer.headdim, 1, 64)
    gbs = nbytes / per_launch / 1e9
    tflops = flops_ref / per_launch / 1e12
    traffic = _traffic_from_profile(os.path.join(ROOT, "profiles", "scan_config2_pmc.txt"))
    log(f"prefill scan: {per_launch * 1e3:.3f} ms/launch, {tokens / per_launch:.4e} tok/s, "
        f"{gbs:.0f} GB/s, {tflops:.1f} TFLOP/s (C_ref=256)")
    return dict(
        per_launch=per_launch, tokens=tokens, t_total=t_scan,
        roofline=dict(bound="hbm", achieved=round(gbs, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                      frac=round(gbs / HBM_PEAK_GBS, 4), traffic=traffic,
                      kernel="m3_scan_fwd: m3::prep_kernel<__bf16> + "
                             "m3::scan16_kernel<__bf16, false>",
                      us_per_launch=round(per_launch * 1e6, 2), bytes_per_launch=nbytes),
        roofline_mfma=dict(bound="mfma", achieved=round(tflops, 1), peak=MFMA_BF16_PEAK_TFLOPS,
                           unit="TFLOP/s", frac=round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
                           flops_per_launch_at_c256=flops_ref,
                           flops_per_launch_at_kernel_chunk64=flops_own),
        forward=dict(tok_s=round(tokens / (t_fwd / FWD_ITERS), 1),
                     ms_per_forward=round(t_fwd / FWD_ITERS * 1e3, 3), iters=FWD_ITERS),
        proj=proj_size)


def step_kernel_name(pairs, rank):
    """The kernel m3_step dispatches for the model's bf16 decode step (N 128, P 64, 32 angles)."""
    if rank == 1:
        return "m3::step128_kernel<__bf16, 1, 8, true>"
    if rank in (2, 4):
        return f"m3::step_mma_kernel<__bf16, {rank}, true>"
    return f"m3::step_kernel<__bf16, {rank}>"


def bench_decode(batch, steps, log, rank=1, prefix=2048):
    from mamba3_amd import Mamba3, ops

    dev = torch.device("cuda:0")
    torch.manual_seed(3)
    model = Mamba3(2048, d_state=128, depth=24, mimo_rank=rank).eval()
    model = model.to(device=dev, dtype=torch.bfloat16)
    gen = torch.Generator(device=dev).manual_seed(3)
    mixer = model.layers[0].mixer
    with torch.inference_mode():
        x = torch.randn(batch, prefix, 2048, device=dev, dtype=torch.bfloat16, generator=gen)
        _, cache = model.prefill(x)
        del x
        decoder = model.cuda_graph(batch_size=batch)
        for layer_cache, src in zip(decoder.cache, cache):
            for dst, s in zip(layer_cache, src):
                dst.copy_(s)
        del cache
        nxt = torch.randn(steps, batch, 1, 2048, device=dev, dtype=torch.bfloat16,
                          generator=gen)
        decoder(nxt[0])
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        for i in range(steps):
            decoder.input.copy_(nxt[i])
            decoder.replay()
        end.record()
        torch.cuda.synchronize()
        t = start.elapsed_time(end) / 1000.0
        # the step kernel alone, in place on the decoder's caches: step i updates layer
        # i % depth with that layer's projection, so the timed steps stream every layer's state
        # in turn, as the decoder does (24 distinct caches; at B = 64 they are 24 x 134 MB,
        # beyond the 256 MB Infinity Cache, so the bytes come from HBM)
        depth = len(model.layers)
        projs = [layer.mixer.in_proj(layer.norm(nxt[0])) for layer in model.layers]
        mixers = [layer.mixer for layer in model.layers]
        iters = 2 * depth

        def step_kernel(i):
            ops.step_projection(projs[i % depth], mixers[i % depth], decoder.cache[i % depth],
                                inplace=True)

        if batch * mixer.nheads >= 8192:
            # eager calls: the launch is GPU-bound at this size (at 1024 pairs a 10 us kernel
            # would time the host's launch rate instead)
            for i in range(3):
                step_kernel(i)
            count = iter(range(10 ** 9))
            t_k = _events_time(lambda: step_kernel(next(count)), iters) / iters
        else:
            # small batches: eager calls would time the host, so a captured graph of
            # back-to-back steps, as the decoder runs them
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                for i in range(3):
                    step_kernel(i)
            torch.cuda.current_stream().wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                for i in range(iters):
                    step_kernel(i)
            graph.replay()
            torch.cuda.synchronize()
            t_k = _events_time(graph.replay, 5) / (5 * iters)
    nb = decode_bytes_per_layer_row(mixer.nheads, mixer.headdim, 128, mixer.num_angles,
                                    rank) * batch
    gbs = nb / t_k / 1e9
    tok_s = steps * batch / t
    log(f"decode B={batch} R={rank}: {t / steps * 1e3:.3f} ms/step, {tok_s:.1f} tok/s; "
        f"step kernel {t_k * 1e6:.1f} us, {gbs:.0f} GB/s")
    # HBM bytes per launch from the committed counter summary (rank 1 at B = 256 only)
    name = ("step_decode_b256_pmc.txt" if (rank, batch) == (1, 256)
            else f"step_decode_b{batch}_rank{rank}_pmc.txt")
    traffic = _traffic_from_profile(os.path.join(ROOT, "profiles", name),
                                    key="traffic_bytes_per_launch:")
    return dict(batch=batch, rank=rank, steps=steps, tok_s=round(tok_s, 1),
                ms_per_step=round(t / steps * 1e3, 4),
                step_kernel=dict(bound="hbm", achieved=round(gbs, 1), peak=HBM_PEAK_GBS,
                                 unit="GB/s", frac=round(gbs / HBM_PEAK_GBS, 4), traffic=traffic,
                                 us_per_launch=round(t_k * 1e6, 2), bytes_per_launch=nb,
                                 kernel=step_kernel_name(batch * mixer.nheads, rank)))


def bench_prefill_config(name, d_model, depth, rank, causal, shape, seed, log, iters=5):
    """Forward throughput of a BASELINE config under bf16 autocast (and one layer's scan call)."""
    from mamba3_amd import Mamba3, ops

    dev = torch.device("cuda:0")
    torch.manual_seed(seed)
    model = Mamba3(d_model, d_state=128, depth=depth, mimo_rank=rank, causal=causal).eval()
    x = torch.randn(*shape)
    model, x = model.to(dev), x.to(dev)
    batch, length = shape[0], shape[1]
    mixer = model.layers[0].mixer
    out = {}
    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.bfloat16):
        # the scan call at steady state (50 warmup launches, as the headline line), then the
        # forward after two warmup passes
        proj = mixer.in_proj(model.layers[0].norm(x))
        call = ops.ScanCall(proj, mixer, chunk_size=mixer.inference_chunk_size)
        for _ in range(50):
            call.launch()
        ts = _events_time(call.launch, 10 * iters) / (10 * iters)
        tp = None
        if not causal:
            # the layer's two directions as the model runs them: the reverse call on a side
            # stream (default priority) concurrent with the forward one, joined after both
            # (each call's segments sized for the two calls' combined grid, as the model's)
            fcall = ops.ScanCall(proj, mixer, chunk_size=mixer.inference_chunk_size,
                                 concurrent=2)
            rcall = ops.ScanCall(proj, mixer, chunk_size=mixer.inference_chunk_size,
                                 reverse=True, concurrent=2)
            main, side = torch.cuda.current_stream(dev), torch.cuda.Stream(device=dev)

            def pair():
                side.wait_stream(main)
                with torch.cuda.stream(side):
                    rcall.launch()
                fcall.launch()
                main.wait_stream(side)

            for _ in range(20):
                pair()
            tp = _events_time(pair, 10 * iters) / (10 * iters)
            del fcall, rcall
        del call, proj
        for _ in range(2):
            model(x)
        t = _events_time(lambda: model(x), iters) / iters
        out["forward_tok_s"] = round(batch * length / t, 1)
        out["ms_per_forward"] = round(t * 1e3, 3)
    c_ref = 256 if rank == 1 else 32
    flops = prefill_flops(batch, length, mixer.nheads, 128, mixer.headdim, rank, c_ref)
    nbytes = prefill_bytes(batch, length, d_model, mixer.in_proj.weight.shape[0])
    # the binding roof: arithmetic intensity at the reference chunk against the ridge
    # (~315 flop/B): rank 1 sits below it (HBM), rank 4 above it (MFMA)
    mfma_bound = flops / nbytes > MFMA_BF16_PEAK_TFLOPS / HBM_PEAK_GBS * 1e3
    achieved = flops / ts / 1e12 if mfma_bound else nbytes / ts / 1e9
    peak = MFMA_BF16_PEAK_TFLOPS if mfma_bound else HBM_PEAK_GBS
    tag = name.replace(" ", "")
    out["scan_call"] = dict(
        us=round(ts * 1e6, 1), tok_s=round(batch * length / ts, 1),
        hbm_frac=round(nbytes / ts / 1e12 / (HBM_PEAK_GBS / 1e3), 4),
        mfma_frac_at_cref=round(flops / ts / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
        # one ScanCall is one direction; a bidirectional layer runs two of them concurrently
        directions=1, layer_directions=1 if causal else 2,
        roofline=dict(bound="mfma" if mfma_bound else "hbm", achieved=round(achieved, 1),
                      peak=peak, unit="TFLOP/s" if mfma_bound else "GB/s",
                      frac=round(achieved / peak, 4),
                      traffic=_traffic_from_profile(
                          os.path.join(ROOT, "profiles", f"scan_{tag}_pmc.txt")),
                      bytes_per_launch=nbytes, flops_per_launch_at_cref=flops))
    if tp is not None:
        # both directions of the layer, concurrent: B L tokens scanned forward and backward
        out["scan_call"]["both_directions"] = dict(
            us=round(tp * 1e6, 1), layer_tok_s=round(batch * length / tp, 1),
            hbm_frac=round(2 * nbytes / tp / 1e12 / (HBM_PEAK_GBS / 1e3), 4),
            vs_two_single_calls=round(tp / (2 * ts), 4))
    log(f"{name}: forward {t * 1e3:.2f} ms ({out['forward_tok_s']:.4e} tok/s); one layer's "
        f"scan call {ts * 1e6:.1f} us" +
        (f", both directions concurrently {tp * 1e6:.1f} us" if tp is not None else ""))
    del model, x
    torch.cuda.empty_cache()
    return out


def bench_chunk_state(log, batch=8, heads=32, width=256, rank=1, n=128, p=64):
    """The standalone per-chunk state update (``m3_chunk_state``) at config 2's chunk shape:
    one chunk of ``width`` tokens for every (batch, head), bf16 k / values, FP32 state. The
    timed calls replay one ~42 MB input set, which stays in the 256 MB Infinity Cache: the
    line reports cache-resident bandwidth (``resident``), not an HBM roof."""
    from mamba3_amd import ops

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(5)
    k = torch.randn(batch, heads, width, rank, n, device=dev, generator=gen).to(torch.bfloat16)
    v = torch.randn(batch, heads, width, rank, p, device=dev, generator=gen).to(torch.bfloat16)
    cum = -torch.rand(batch, heads, width, device=dev, generator=gen).cumsum(-1) * 0.01
    scale = torch.rand(batch, heads, width, device=dev, generator=gen) * 0.1
    state = torch.randn(batch, heads, p, n, device=dev, generator=gen)
    out = torch.empty_like(state)

    def call():
        ops.chunk_state(k, v, cum, scale, state, out, width=width, rank=rank)

    # one call is shorter than its host-side launch path, so the timed calls replay a graph
    with torch.inference_mode():
        for _ in range(50):
            call()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(50):
                call()
        graph.replay()
        t = _events_time(graph.replay, 4) / 200
    nbytes = (batch * heads * width * rank * (n + p) * 2 + batch * heads * width * 8
              + 2 * batch * heads * p * n * 4)
    gbs = nbytes / t / 1e9
    log(f"chunk_state B={batch} H={heads} W={width}: {t * 1e6:.2f} us, {gbs:.0f} GB/s")
    return dict(us=round(t * 1e6, 2), bytes=nbytes, achieved=round(gbs, 1), unit="GB/s",
                resident="infinity cache (one 42 MB input set replayed)",
                traffic=_traffic_from_profile(
                    os.path.join(ROOT, "profiles", "chunk_state_config2_pmc.txt")),
                kernel="m3::chunk_state_mma_kernel<__bf16>",
                shape=f"[{batch}, {heads}] x {width} tokens, R={rank}, N={n}, P={p}")


def bench_hook_step(log, batch=256, heads=32, p=64, n=128, rank=1):
    """The reference's decode hook boundary (``fused_step``: head-expanded, biased, unrotated
    q / k [B, H, R, N] bf16, value / gate [B, H, P], FP32 adt / dt, the angle rates, cache tensors
    updated out of place) at B=256 with 32 heads of config 2's shape: the step kernel's generic
    form. Bytes: the FP32 state read and written plus the per-row vectors."""
    from mamba3_amd import ops

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(7)
    bf = torch.bfloat16
    s = n // 4

    def rnd(*shape, dtype=torch.float32):
        return torch.randn(*shape, device=dev, generator=gen).to(dtype)

    dt = torch.rand(batch, heads, device=dev, generator=gen) * 0.1 + 0.001
    inp = dict(q=rnd(batch, heads, rank, n, dtype=bf), k=rnd(batch, heads, rank, n, dtype=bf),
               value=rnd(batch, heads, p, dtype=bf), gate=rnd(batch, heads, p, dtype=bf),
               adt=-0.5 * dt, dt=dt, trap_logits=rnd(batch, heads, dtype=bf),
               angle_rate=rnd(batch, s, dtype=bf), D=rnd(heads))
    if rank > 1:
        inp.update(mimo_x=rnd(heads, rank, p) / rank, mimo_z=rnd(heads, rank, p),
                   mimo_out=rnd(heads, rank, p) / rank)
    cache = (rnd(batch, heads, s), rnd(batch, heads, p, n), rnd(batch, heads, rank, n, dtype=bf),
             rnd(batch, heads, p, dtype=bf))

    def call():
        ops.fused_step(**inp, cache=cache)

    with torch.inference_mode():
        for _ in range(50):
            call()
        t = _events_time(call, 50) / 50
    rows = batch * heads
    # state in / out, q / k, prev_k / k_out, value / gate / prev_value / value_out / y, phase
    # in / out
    nbytes = rows * (2 * p * n * 4 + 2 * 2 * rank * n * 2 + 2 * 2 * rank * n * 2 + 5 * p * 2
                     + 2 * s * 4)
    gbs = nbytes / t / 1e9
    log(f"hook step (fused_step) B={batch} H={heads} R={rank}: {t * 1e6:.1f} us, {gbs:.0f} GB/s")
    return dict(us=round(t * 1e6, 1), tok_s=round(batch / t, 1), bytes=nbytes, bound="hbm",
                achieved=round(gbs, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                frac=round(gbs / HBM_PEAK_GBS, 4))


def bench_hook_scan(log, batch=8, length=8192, heads=32, p=64, n=128):
    """The reference's scan hook boundary (``mamba3_scan``: normed q / k, head-expanded value /
    gate, FP32 adt / dt, trap logits and the materialized phases [B, L, H, S] FP32) at config 2's
    shape, bf16: the generic kernel path, which reads the inputs as given."""
    from mamba3_amd import ops

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(6)
    bf = torch.bfloat16
    s = n // 4

    def rnd(*shape, dtype=torch.float32):
        return torch.randn(*shape, device=dev, generator=gen).to(dtype)

    dt = torch.rand(batch, length, heads, device=dev, generator=gen) * 0.1 + 0.001
    inp = dict(q=rnd(batch, length, 1, 1, n, dtype=bf), k=rnd(batch, length, 1, 1, n, dtype=bf),
               value=rnd(batch, length, heads, p, dtype=bf),
               gate=rnd(batch, length, heads, p, dtype=bf),
               adt=-dt * torch.rand(batch, length, heads, device=dev, generator=gen), dt=dt,
               trap_logits=rnd(batch, length, heads, dtype=bf), D=rnd(heads),
               phase=(torch.rand(batch, length, heads, s, device=dev, generator=gen) * 2 - 1) * 6.28,
               q_bias=1 + 0.1 * rnd(heads, 1, n), k_bias=1 + 0.1 * rnd(heads, 1, n))

    def call():
        ops.mamba3_scan(**inp, chunk_size=256)

    with torch.inference_mode():
        for _ in range(50):  # past the clock ramp of sustained load
            call()
        t = _events_time(call, 50) / 50
    tokens = batch * length
    nbytes = (tokens * (2 * n * 2 + 2 * heads * p * 2 + heads * (4 + 4 + 2) + heads * s * 4)
              + tokens * heads * p * 2)
    gbs = nbytes / t / 1e9
    log(f"hook scan (mamba3_scan, given phases) {batch}x{length}: {t * 1e6:.1f} us, "
        f"{tokens / t:.4e} tok/s, {gbs:.0f} GB/s")
    return dict(us=round(t * 1e6, 1), tok_s=round(tokens / t, 1), bytes=nbytes, bound="hbm",
                achieved=round(gbs, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                frac=round(gbs / HBM_PEAK_GBS, 4))


def bench_cpu(log, batch=8, length=8192):
    """The CPU oracle (portable-path restatement) on the prefill scan, ``x[batch, length]``."""
    from oracle import portable as op

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    torch.manual_seed(1)
    params = op.init_params(1024, d_state=128, depth=1, mimo_rank=1)
    dims = op.Dims(1024, 128, 1)
    x = torch.randn(batch, length, 1024)
    pre = "layers.0.mixer."
    with torch.inference_mode():
        proj = torch.nn.functional.linear(op.rms_norm(x, params["layers.0.norm.weight"]),
                                          params[pre + "in_proj.weight"])

        def hot_path():
            sizes = dims.split_sizes
            z, xv, b, c, ddt, da, trap, ang = torch.split(proj, sizes, dim=-1)
            hh, pp, nn_ = dims.nheads, dims.headdim, dims.d_state
            z = z.reshape(batch, length, hh, pp)
            xv = xv.reshape(batch, length, hh, pp)
            k = op.rms_norm(b.reshape(batch, length, 1, 1, nn_), params[pre + "B_norm.weight"])
            q = op.rms_norm(c.reshape(batch, length, 1, 1, nn_), params[pre + "C_norm.weight"])
            dt = torch.nn.functional.softplus(ddt + params[pre + "dt_bias"])
            adt = (-op.heavy_tail(da)).clamp(max=-op.A_FLOOR) * dt
            phase = op.phase_scan(ang, dt)
            return op.ssd_scan(q.permute(0, 1, 3, 2, 4), k.permute(0, 1, 3, 2, 4), xv, z, adt,
                               dt, trap, params[pre + "D"], chunk_size=256, phase=phase,
                               q_bias=params[pre + "C_bias"], k_bias=params[pre + "B_bias"])

        hot_path()
        times = []
        for _ in range(3):
            t0 = time.perf_counter()
            hot_path()
            times.append(time.perf_counter() - t0)
    t = sorted(times)[1]
    tok_s = batch * length / t
    log(f"cpu oracle: {t:.3f} s for {batch}x{length} tokens on {cores} threads -> "
        f"{tok_s:.1f} tok/s")
    return dict(value=round(tok_s, 1), unit="tok/s", cores=cores, kind="port",
                sample=(f"the scan hot path (B/C RMSNorm, dt/A, phase, chunked SSD at chunk 256) "
                        f"of config 2's mixer on x[{batch}, {length}, 1024] in FP32, median of 3 after "
                        f"1 warmup"))


def bench_cpu_decode(log, batch=256, steps=3):
    """The CPU oracle on the decode step's hot path: one config-4 layer (d_model 2048, R = 1) at
    ``batch`` rows, FP32, from the raw ``in_proj`` output (the GEMMs are not timed, as on the
    GPU's step-kernel line): split, B/C RMSNorm, dt/A, head biases, phase advance, rotation and
    the exact update and readout."""
    from oracle import portable as op

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    torch.manual_seed(3)
    dims = op.Dims(2048, 128, 1)
    params = op.init_params(2048, d_state=128, depth=1, mimo_rank=1)
    pre = "layers.0.mixer."
    hh, pp, nn_ = dims.nheads, dims.headdim, dims.d_state
    cache = list(op.zero_cache(dims, batch, torch.float32))
    cache[1] = torch.randn(batch, hh, pp, nn_) * 0.1
    with torch.inference_mode():
        projs = [torch.nn.functional.linear(
            op.rms_norm(torch.randn(batch, 2048), params["layers.0.norm.weight"]),
            params[pre + "in_proj.weight"]) for _ in range(steps + 1)]

        def hot_path(proj, cache):
            z, xv, b, c, ddt, da, trap, ang = torch.split(proj, dims.split_sizes, dim=-1)
            k = op.rms_norm(b.reshape(batch, 1, 1, nn_), params[pre + "B_norm.weight"])
            q = op.rms_norm(c.reshape(batch, 1, 1, nn_), params[pre + "C_norm.weight"])
            q = q.expand(batch, hh, 1, nn_) + params[pre + "C_bias"]
            k = k.expand(batch, hh, 1, nn_) + params[pre + "B_bias"]
            dt = torch.nn.functional.softplus(ddt + params[pre + "dt_bias"])
            adt = (-op.heavy_tail(da)).clamp(max=-op.A_FLOOR) * dt
            phase = torch.fmod(cache[0] + op.phase_increment(ang, dt), op.TWO_PI)
            q, k = op.rotate(q[:, None], k[:, None], phase[:, None], mimo=False)
            return op.step_update(q[:, 0], k[:, 0], xv.reshape(batch, hh, pp),
                                  z.reshape(batch, hh, pp), adt, dt, trap, params[pre + "D"],
                                  (phase, cache[1], cache[2], cache[3]))

        _, cache = hot_path(projs[0], cache)
        times = []
        for i in range(steps):
            t0 = time.perf_counter()
            _, cache = hot_path(projs[i + 1], cache)
            times.append(time.perf_counter() - t0)
    t = sorted(times)[len(times) // 2]
    tok_s = batch / (24 * t)
    log(f"cpu oracle decode: {t * 1e3:.1f} ms per layer step at B={batch} on {cores} threads -> "
        f"{tok_s:.1f} tok/s over 24 layers (step hot path only)")
    return dict(value=round(tok_s, 1), unit="tok/s", cores=cores, kind="port",
                ms_per_layer_step=round(t * 1e3, 2),
                sample=(f"the decode step's hot path (split, B/C RMSNorm, dt/A, biases, phase, "
                        f"rotation, update and readout; no projection GEMMs) of one config-4 layer "
                        f"(d_model 2048, R 1) at B={batch} in FP32, median of {steps} steps after "
                        f"1 warmup; value = B / (24 x per-layer time), to set beside "
                        f"decode.step_kernel"))


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # The headline call's timed steps follow the forward line's 30 passes (same kernels), so a
    # few warmup calls suffice; 50 are the default
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--decode-batch", type=int, default=256)
    ap.add_argument("--decode-steps", type=int, default=512)
    ap.add_argument("--decode-rank", type=int, default=1, choices=(1, 2, 4),
                    help="MIMO rank of the decode line's model (config 4 runs 1 and 4)")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-batch", type=int, default=8)
    ap.add_argument("--cpu-tokens", type=int, default=8192)
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the default extra lines (configs 3, 5 and 5 long, decode R=4 "
                         "B=256, R=1 B=64 and R=1 B=1)")
    ap.add_argument("--extra", action="store_true",
                    help="also measure config 4 at more B and R, the chunk-state update and "
                         "the hook boundaries")
    ap.add_argument("--extra-only", choices=("config3", "config5", "decode",
                                             "chunk_state", "hook", "hook_step"),
                    help="with --extra: measure only this one of the extra configurations")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also run a plain 1 GiB device copy (calibrates PMC byte counters)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: the Mamba-3 hot path of this build runs on a single "
              "MI355X (the (batch, head) recurrences shard over GPUs without communication; a "
              "multi-GPU run is not part of this build).", file=sys.stderr)
        sys.exit(2)

    def log(msg):
        print(msg, file=sys.stderr, flush=True)

    # The headline call is prepared first. The default extra lines (5 and 5
    # long and three more decode points) run next, then the config-2 forward line, and the
    # headline scan calls are timed right after it: they then run at the clocks of sustained
    # load of the same kernels, as in a prefill loop, not in the clock ramp that follows a
    # change of workload.
    prep = prepare_prefill()
    extra = {}
    if not args.no_extra:
        if not args.no_decode:
            extra["config4_decode_r4_b256"] = bench_decode(256, args.decode_steps, log, rank=4)
            extra["config4_decode_r1_b64"] = bench_decode(64, args.decode_steps, log, rank=1)
            extra["config4_decode_r1_b1"] = bench_decode(1, args.decode_steps, log, rank=1)
        extra["config5_bidir_16x2048"] = bench_prefill_config(
            "config 5", 768, 12, 1, False, (16, 2048, 768), 4, log)
        extra["config5_bidir_1x65536"] = bench_prefill_config(
            "config 5 long", 768, 12, 1, False, (1, 65536, 768), 4, log, iters=2)
        extra["config3_mimo_prefill"] = bench_prefill_config(
            "config 3", 1024, 4, 4, True, (8, 4096, 1024), 2, log)
    pre = bench_prefill(prep, args.steps, args.warmup, log, copy_probe=args.copy_probe)
    del prep
    torch.cuda.empty_cache()
    decode = None
    if not args.no_decode:
        decode = bench_decode(args.decode_batch, args.decode_steps, log, rank=args.decode_rank)
    if args.extra:
        runs = {
            "config3_mimo_prefill": ("config3", lambda: bench_prefill_config(
                "config 3", 1024, 4, 4, True, (8, 4096, 1024), 2, log)),
            "config5_bidir_16x2048": ("config5", lambda: bench_prefill_config(
                "config 5", 768, 12, 1, False, (16, 2048, 768), 4, log)),
            "config4_decode": ("decode", lambda: [
                bench_decode(b, args.decode_steps, log, rank=r)
                for b, r in ((64, 4), (1, 4), (32, 1), (16, 1))]),
            "chunk_state_config2": ("chunk_state", lambda: bench_chunk_state(log)),
            "hook_scan_config2": ("hook", lambda: bench_hook_scan(log)),
            "hook_step_b256": ("hook_step", lambda: [bench_hook_step(log, rank=r) for r in (1, 4)]),
        }
        extra.update({name: run() for name, (key, run) in runs.items()
                      if args.extra_only in (None, key)})
    cpu = None if args.no_cpu else bench_cpu(log, args.cpu_batch, args.cpu_tokens)
    cpu_decode = None if args.no_cpu or args.no_decode else bench_cpu_decode(log)
    value = pre["tokens"] / pre["per_launch"]
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(pre["per_launch"] * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) inputs, random-init weights)",
        "config": {"workload": "config 2: SISO prefill scan (m3_scan_fwd) of "
                               "Mamba3(1024, 128, depth=1, mimo_rank=1), x[8, 8192, 1024], "
                               "bf16 autocast, in_proj output resident in HBM",
                   "global_batch": 8, "seq_len": 8192, "parallelism": "none (1 GPU)"},
        "roofline": pre["roofline"],
        "roofline_mfma": pre["roofline_mfma"],
        "forward": pre["forward"],
        "decode": decode,
        "cpu_baseline": cpu,
        "cpu_baseline_decode": cpu_decode,
    }
    if extra:
        line["extra_configs"] = extra
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

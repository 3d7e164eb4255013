"""The drop-in ``Mamba3`` API on the CPU: signature, parameters, validation, no fallback.

Model-level numerics need the GPU (``test_gpu_model.py``); here the product must match
the reference's construction (names, shapes, RNG order via golden checksums) and its
validation errors, and must refuse to run the hot path on CPU tensors.
"""

from __future__ import annotations

import inspect

import numpy as np
import pytest
import torch

import mamba3_amd
from conftest import golden
from mamba3_amd import Mamba3, ops


def test_only_mamba3_is_public_and_constructor_is_small():
    """Reference tests/test_model.py:31-39."""
    assert mamba3_amd.__all__ == ["Mamba3"]
    assert list(inspect.signature(Mamba3).parameters) == [
        "d_model", "d_state", "depth", "mimo_rank", "causal"]


def test_constructor_validation():
    """Reference tests/test_model.py:42-52."""
    with pytest.raises(ValueError, match="d_model"):
        Mamba3(0)
    with pytest.raises(ValueError, match="at least 4"):
        Mamba3(16, d_state=2)
    with pytest.raises(ValueError, match="divisible by 4"):
        Mamba3(16, d_state=10, mimo_rank=4)
    with pytest.raises(ValueError, match="depth"):
        Mamba3(16, depth=0)
    with pytest.raises(ValueError, match="mimo_rank"):
        Mamba3(16, mimo_rank=0)


@pytest.mark.parametrize("rank", [1, 4])
def test_has_canonical_mamba3_parameters(rank):
    """Reference tests/test_model.py:55-75."""
    mixer = Mamba3(64, depth=1, mimo_rank=rank).layers[0].mixer
    assert (mixer.d_state, mixer.d_inner, mixer.headdim, mixer.nheads, mixer.num_angles) == (
        128, 128, 64, 2, 32)
    assert mixer.in_proj.weight.shape == (2 * 128 + 2 * 128 * rank + 3 * 2 + 32, 64)
    assert mixer.B_bias.shape == mixer.C_bias.shape == (2, rank, 128)
    assert not hasattr(mixer, "conv1d") and not hasattr(mixer, "A_log")
    if rank == 1:
        assert mixer.mimo_x is None
    else:
        assert mixer.mimo_x.shape == (2, rank, 64)
    views = ops.split_projection(mixer.in_proj(torch.randn(1, 3, 64)), mixer)
    assert views["q"].shape == views["k"].shape == (1, 3, 1, rank, 128)
    assert views["x"].shape == views["z"].shape == (1, 3, 2, 64)
    assert views["dt"].shape == views["a"].shape == views["trap"].shape == (1, 3, 2)
    assert views["angles"].shape == (1, 3, 32)


def test_canonical_initialization():
    """Reference tests/test_model.py:78-92."""
    mixer = Mamba3(32, d_state=8, depth=1, mimo_rank=4).layers[0].mixer
    for t, v in ((mixer.B_bias, 1.0), (mixer.C_bias, 1.0), (mixer.D, 1.0), (mixer.mimo_x, 0.25),
                 (mixer.mimo_z, 1.0), (mixer.mimo_out, 0.25)):
        torch.testing.assert_close(t, torch.full_like(t, v))
    dt = torch.nn.functional.softplus(mixer.dt_bias)
    assert (dt >= 0.001).all() and (dt <= 0.1).all()


def _checksums_match(data, model):
    names = [n for n, _ in model.named_parameters()]
    assert names == [str(n) for n in data["param_order"]]
    for name, p in model.named_parameters():
        v = p.detach().double()
        got = np.array([v.sum().item(), v.square().sum().item(), *v.flatten()[:4].tolist()]
                       + [0.0] * max(0, 4 - v.numel()))
        np.testing.assert_allclose(got, data[f"param/{name}"], rtol=1e-12, atol=1e-12,
                                   err_msg=name)


@pytest.mark.parametrize("rank", [1, 4])
def test_seeded_parameters_equal_the_reference(rank):
    """Same names, order and values under torch.manual_seed as the reference."""
    torch.manual_seed(100 + rank)
    _checksums_match(golden(f"model_r{rank}_f32.npz"), Mamba3(64, d_state=16, depth=2,
                                                              mimo_rank=rank))
    torch.manual_seed(40 + rank)
    _checksums_match(golden(f"bidir_r{rank}.npz"),
                     Mamba3(16, d_state=8, depth=2, mimo_rank=rank, causal=False))


def test_config1_parameters_equal_the_reference():
    torch.manual_seed(0)
    _checksums_match(golden("config1.npz"), Mamba3(256, d_state=128, depth=6, mimo_rank=1))


def test_state_dict_loads_reference_names():
    model = Mamba3(32, d_state=8, depth=2, mimo_rank=4, causal=False)
    keys = set(model.state_dict())
    for i in range(2):
        for name in ("norm.weight", "mixer.in_proj.weight", "mixer.B_norm.weight",
                     "mixer.C_norm.weight", "mixer.B_bias", "mixer.C_bias", "mixer.dt_bias",
                     "mixer.D", "mixer.mimo_x", "mixer.mimo_z", "mixer.mimo_out",
                     "mixer.out_proj.weight", "mixer.direction_logit"):
            assert f"layers.{i}.{name}" in keys
    assert "norm_f.weight" in keys


def test_empty_inputs_need_no_kernel():
    """Reference tests/test_model.py:15-28 (the empty cases)."""
    model = Mamba3(d_model=24, d_state=8, depth=2)
    assert model(torch.empty(0, 5, 24)).shape == (0, 5, 24)
    assert model(torch.empty(2, 0, 24)).shape == (2, 0, 24)
    with pytest.raises(ValueError, match="expected"):
        model(torch.empty(2, 5, 7))


def test_cpu_hot_path_fails_loudly():
    """No CPU fallback: the hot path refuses CPU tensors."""
    model = Mamba3(16, d_state=8, depth=1).eval()
    with torch.inference_mode(), pytest.raises(RuntimeError, match="ROCm"):
        model(torch.randn(1, 4, 16))
    with torch.inference_mode(), pytest.raises(RuntimeError, match="ROCm"):
        model.step(torch.randn(1, 1, 16))
    q = torch.randn(1, 3, 1, 1, 8)
    v = torch.randn(1, 3, 2, 4)
    s = torch.randn(1, 3, 2)
    with pytest.raises(RuntimeError, match="ROCm"):
        ops.mamba3_scan(q, q, v, v, -s.abs(), s.abs(), s, torch.ones(2))


def test_autograd_use_fails_loudly():
    model = Mamba3(16, d_state=8, depth=1)
    with pytest.raises(RuntimeError, match="no backward"):
        model(torch.randn(1, 4, 16))


def test_step_validates_input_and_cache():
    """Reference tests/test_model.py:276-293 (validation happens before the kernels)."""
    model = Mamba3(16, d_state=8, depth=2)
    with pytest.raises(ValueError, match="batch, 1"):
        model.step(torch.randn(2, 3, 16))
    with pytest.raises(ValueError, match="cache for 2"):
        model.step(torch.randn(2, 1, 16), cache=[])
    mixer = model.layers[0].mixer
    cache = [mixer.allocate_cache(2, device=torch.device("cpu"), dtype=torch.float32)
             for _ in range(2)]
    cache[0] = (cache[0][0], cache[0][1], cache[0][2][:1], cache[0][3])
    with torch.inference_mode(), pytest.raises(ValueError, match="cache shapes"):
        model.step(torch.randn(2, 1, 16), cache)
    with pytest.raises(ValueError, match="non-empty"):
        model.prefill(torch.empty(2, 0, 16))


def test_bidirectional_rejects_caches_prefill_and_step():
    """Reference tests/test_model.py:153-161."""
    model = Mamba3(16, d_state=8, depth=1, causal=False)
    with pytest.raises(ValueError, match="causal"):
        model.prefill(torch.randn(1, 4, 16))
    with pytest.raises(ValueError, match="causal"):
        model.step(torch.randn(1, 1, 16))
    with pytest.raises(ValueError, match="causal"):
        model.layers[0].mixer(torch.randn(1, 4, 16), return_cache=True)
    assert model.layers[0].mixer.direction_logit is not None


def test_scan_validation_messages_mirror_the_reference():
    q = torch.randn(1, 3, 1, 1, 8)
    v = torch.randn(1, 3, 2, 4)
    s = torch.randn(1, 3, 2)
    with pytest.raises(ValueError, match="matching"):
        ops.mamba3_scan(q, q[:, :2], v, v, s, s, s, torch.ones(2))
    with pytest.raises(ValueError, match="D must have shape"):
        ops.mamba3_scan(q, q, v, v, s, s, s, torch.ones(3))
    with pytest.raises(ValueError, match="chunk_size"):
        ops.mamba3_scan(q, q, v, v, s, s, s, torch.ones(2), chunk_size=0)
    with pytest.raises(ValueError, match="SISO"):
        ops.mamba3_scan(q, q, v, v, s, s, s, torch.ones(2), mimo_x=torch.ones(2, 1, 4))


def test_set_chunk_sizes_and_compile_are_accepted():
    model = Mamba3(16, d_state=8, depth=2)
    assert model.set_chunk_sizes(training=32, inference=64) is model
    assert all(layer.mixer.inference_chunk_size == 64 for layer in model.layers)
    with pytest.raises(ValueError):
        model.set_chunk_sizes(inference=0)
    assert model.compile() is model
    assert model.compile_layers() is model


def test_graph_decoder_validate_sees_moved_storage():
    """The graph decoder's staleness check compares what the reference's
    ``_parameter_signature`` compares (``model.py:763-774``): identity, version, data pointer,
    device, dtype and shape. ``p.data = ...`` and ``Module.to(dtype)`` keep the Parameter object
    and its version, so a check of those two alone passes a graph that reads freed weights.
    The decoder's capture needs a GPU; its check does not, so it runs here on a decoder whose
    capture record is taken from a CPU model."""
    from mamba3_amd.model import _HipGraphDecoder, _storage_signature

    def decoder_for(model):
        dec = object.__new__(_HipGraphDecoder)
        dec.model = model
        dec._captured = [_storage_signature(w) for w in model.parameters()]
        return dec

    model = Mamba3(16, d_state=8, depth=1)
    dec = decoder_for(model)
    dec.validate()
    weight = model.layers[0].mixer.in_proj.weight
    version = weight._version
    weight.data = weight.data.clone()
    assert weight._version == version
    with pytest.raises(RuntimeError, match="recreate"):
        dec.validate()

    dec = decoder_for(model)
    before = list(model.parameters())
    model.to(torch.bfloat16)
    assert all(a is b for a, b in zip(before, model.parameters()))
    with pytest.raises(RuntimeError, match="recreate"):
        dec.validate()

    dec = decoder_for(model)
    with torch.no_grad():
        model.layers[0].mixer.D.add_(1)
    with pytest.raises(RuntimeError, match="recreate"):
        dec.validate()

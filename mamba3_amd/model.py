"""The drop-in ``Mamba3`` module (reference ``mamba3/model.py``, jreoka/mamba3).

Same constructor, parameter names and shapes, parameter-creation order under
``torch.manual_seed``, methods and validation messages as the reference. The hot path
differs: after the ``in_proj`` GEMM, each mixer hands the raw projection to one HIP
kernel (``ops.scan_projection`` / ``ops.step_projection``). That kernel does the B/C
RMSNorm, dt / A, the bounded phase, bias and rotation, and the chunked SSD or the
decode step. ``in_proj`` / ``out_proj`` and the residual RMSNorm stay in torch
(hipBLASLt), except in a decode step of a small batch with 16-bit weights: there both
projections run on ``ops.linear`` (``m3_linear``), the block's RMSNorm fused into
``in_proj`` and its residual add into ``out_proj``.

Scope: inference (``forward``, ``prefill``, ``step``, ``cuda_graph``) on ROCm devices.
Autograd through the mixer and CPU execution raise ``RuntimeError``. ``compile`` and
``compile_layers`` are accepted and leave the module unchanged (no Inductor / Triton).
"""

from __future__ import annotations

import math
import os

import torch
from torch import nn
from torch.nn import functional as F

from . import ops

_EXPANSION = 2
_CANONICAL_HEAD_DIM = 64
_ROPE_FRACTION = 0.5

_LayerCache = tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]


def _default_chunk_sizes(mimo_rank: int) -> tuple[int, int]:
    """Training / inference chunk sizes of the reference (``model.py:26-37``)."""
    training = 512 if mimo_rank == 1 else max(8, 64 // mimo_rank)
    inference = 256 if mimo_rank == 1 else max(16, 128 // mimo_rank)
    return training, inference


_SIDE_STREAMS: dict[torch.device, torch.cuda.Stream] = {}


def _side_stream(device: torch.device) -> torch.cuda.Stream:
    """A second stream per device (default priority) for the reverse scan of a bidirectional
    layer."""
    if device not in _SIDE_STREAMS:
        _SIDE_STREAMS[device] = torch.cuda.Stream(device=device)
    return _SIDE_STREAMS[device]


class _RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float = 1e-5) -> None:
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        y = F.rms_norm(x, (x.shape[-1],), self.weight.to(dtype=x.dtype), self.eps)
        return y.to(dtype=x.dtype)


class _Mamba3Mixer(nn.Module):
    """One Mamba-3 SISO / MIMO mixer; the scan and the step run in the HIP library."""

    def __init__(self, d_model: int, d_state: int, mimo_rank: int, causal: bool = True) -> None:
        super().__init__()
        self.d_model = d_model
        self.d_state = d_state
        self.mimo_rank = mimo_rank
        self.causal = causal
        self.d_inner = _EXPANSION * d_model
        self.headdim = math.gcd(self.d_inner, _CANONICAL_HEAD_DIM)
        self.nheads = self.d_inner // self.headdim
        self.ngroups = 1
        self.num_angles = int(d_state * _ROPE_FRACTION) // 2
        train_chunk, inference_chunk = _default_chunk_sizes(mimo_rank)
        env_chunk = os.getenv("MAMBA3_CHUNK_SIZE")
        if env_chunk:
            try:
                override = int(env_chunk)
            except ValueError as error:
                raise ValueError("MAMBA3_CHUNK_SIZE must be a positive integer") from error
            if override <= 0:
                raise ValueError("MAMBA3_CHUNK_SIZE must be a positive integer")
            train_chunk = inference_chunk = override
        self.chunk_size = train_chunk
        self.inference_chunk_size = inference_chunk

        projection_size = (2 * self.d_inner + 2 * d_state * self.ngroups * mimo_rank
                           + 3 * self.nheads + self.num_angles)
        # Parameter creation order matches the reference so seeds reproduce its weights:
        # in_proj (RNG), norms, biases, dt_bias (RNG), D, MIMO, out_proj (RNG).
        self.in_proj = nn.Linear(d_model, projection_size, bias=False)
        self.B_norm = _RMSNorm(d_state)
        self.C_norm = _RMSNorm(d_state)
        self.B_bias = nn.Parameter(torch.ones(self.nheads, mimo_rank, d_state))
        self.C_bias = nn.Parameter(torch.ones(self.nheads, mimo_rank, d_state))
        dt = torch.exp(torch.rand(self.nheads) * (math.log(0.1) - math.log(0.001))
                       + math.log(0.001)).clamp_min(1e-4)
        self.dt_bias = nn.Parameter(dt + torch.log(-torch.expm1(-dt)))
        self.dt_bias._no_weight_decay = True
        self.D = nn.Parameter(torch.ones(self.nheads))
        self.D._no_weight_decay = True
        if mimo_rank > 1:
            self.mimo_x = nn.Parameter(
                torch.full((self.nheads, mimo_rank, self.headdim), 1.0 / mimo_rank))
            self.mimo_z = nn.Parameter(torch.ones(self.nheads, mimo_rank, self.headdim))
            self.mimo_out = nn.Parameter(
                torch.full((self.nheads, mimo_rank, self.headdim), 1.0 / mimo_rank))
        else:
            self.register_parameter("mimo_x", None)
            self.register_parameter("mimo_z", None)
            self.register_parameter("mimo_out", None)
        self.out_proj = nn.Linear(self.d_inner, d_model, bias=False)
        if causal:
            self.register_parameter("direction_logit", None)
        else:
            self.direction_logit = nn.Parameter(torch.zeros(d_model))

    def _chunk(self) -> int:
        return (self.chunk_size if self.training and torch.is_grad_enabled()
                else self.inference_chunk_size)

    def _check_inference(self, *tensors: torch.Tensor) -> None:
        params_need_grad = any(p.requires_grad for p in self.parameters())
        if torch.is_grad_enabled() and (params_need_grad or any(t.requires_grad for t in tensors)):
            raise RuntimeError(
                "mamba3_amd implements the inference hot path (forward, prefill, step) and has "
                "no backward; run it under torch.no_grad() or torch.inference_mode()")

    # ---- forward / prefill

    def forward(self, hidden_states: torch.Tensor, cache: _LayerCache | None = None, *,
                return_cache: bool = False):
        if not self.causal and (cache is not None or return_cache):
            raise ValueError("bidirectional Mamba3 does not support caches; "
                             "prefill and step require causal=True")
        self._check_inference(hidden_states)
        proj = self.in_proj(hidden_states)
        if not self.causal:
            # the reverse scan on a side stream, concurrent with the forward one: each direction
            # alone may leave CUs idle in its last round of workgroups
            main = torch.cuda.current_stream(proj.device)
            side = _side_stream(proj.device)
            side.wait_stream(main)
            with torch.cuda.stream(side):
                mixed_r, _, _, _ = ops.scan_projection(proj, self, chunk_size=self._chunk(),
                                                       reverse=True, concurrent=2)
            proj.record_stream(side)
        mixed, state, final_phase, final_k = ops.scan_projection(
            proj, self, cache=cache, want_cache=return_cache and self.causal,
            chunk_size=self._chunk(), concurrent=1 if self.causal else 2)
        output = self.out_proj(mixed.flatten(-2))
        if self.causal:
            if not return_cache:
                return output
            last_value = proj[:, -1, self.d_inner:2 * self.d_inner].unflatten(
                -1, (self.nheads, self.headdim)).clone()
            return output, (final_phase, state, final_k, last_value)
        # Bidirectional (model.py:330-362): the reversed sequence with the same weights. The
        # projection is per token, so in_proj(flip(x)) = flip(in_proj(x)): the reverse scan
        # (launched above) reads this projection backwards and writes its output back in forward
        # order (no flip, no second projection).
        main.wait_stream(side)
        mixed_r.record_stream(main)
        backward = self.out_proj(mixed_r.flatten(-2))
        blend = torch.sigmoid(self.direction_logit).to(dtype=output.dtype)
        return output * blend + backward * (1.0 - blend)

    # ---- decode

    def allocate_cache(self, batch_size: int, *, device: torch.device,
                       dtype: torch.dtype) -> _LayerCache:
        return (
            torch.zeros(batch_size, self.nheads, self.num_angles, device=device,
                        dtype=torch.float32),
            torch.zeros(batch_size, self.nheads, self.headdim, self.d_state, device=device,
                        dtype=torch.float32),
            torch.zeros(batch_size, self.nheads, self.mimo_rank, self.d_state, device=device,
                        dtype=dtype),
            torch.zeros(batch_size, self.nheads, self.headdim, device=device, dtype=dtype),
        )

    def _validate_cache(self, cache: _LayerCache, batch_size: int) -> None:
        if len(cache) != 4:
            raise ValueError("a Mamba-3 layer cache must contain four tensors")
        expected = (
            (batch_size, self.nheads, self.num_angles),
            (batch_size, self.nheads, self.headdim, self.d_state),
            (batch_size, self.nheads, self.mimo_rank, self.d_state),
            (batch_size, self.nheads, self.headdim),
        )
        actual = tuple(tuple(t.shape) for t in cache)
        if actual != expected:
            raise ValueError(f"expected cache shapes {expected}, got {actual}")
        if cache[0].dtype != torch.float32 or cache[1].dtype != torch.float32:
            raise ValueError("phase and SSM cache tensors must be float32")
        device = self.in_proj.weight.device
        if any(t.device != device for t in cache):
            raise ValueError(f"cache tensors must be on {device}")

    def step(self, hidden_states: torch.Tensor, cache: _LayerCache | None, *,
             inplace: bool = False, residual: torch.Tensor | None = None,
             norm: _RMSNorm | None = None):
        """One decode token. ``norm`` (the block's RMSNorm) is applied to ``hidden_states``
        first; with ``residual`` (``[batch, 1, d_model]``) the result is
        ``residual + out_proj(...)``. With 16-bit weights, ``in_proj`` runs on ``ops.linear``
        with the norm fused up to ``ops.DECODE_LINEAR_ROWS`` rows, and ``out_proj`` with the
        residual add fused up to ``ops.DECODE_LINEAR_OUT_ROWS``."""
        if hidden_states.ndim != 3 or hidden_states.shape[1:] != (1, self.d_model):
            raise ValueError(
                f"expected [batch, 1, {self.d_model}], got {tuple(hidden_states.shape)}")
        self._check_inference(hidden_states)
        rows = hidden_states[:, 0]
        small = rows.shape[0] <= ops.DECODE_LINEAR_ROWS
        supported = ops.linear_norm_supported if norm is not None else ops.linear_supported
        if small and supported(rows, self.in_proj.weight):
            proj = ops.linear(rows, self.in_proj.weight,
                              norm_weight=norm.weight if norm is not None else None,
                              norm_eps=norm.eps if norm is not None else ops.NORM_EPS)
            proj = proj.unsqueeze(1)
        else:
            proj = self.in_proj(norm(hidden_states) if norm is not None else hidden_states)
        if cache is None:
            cache = self.allocate_cache(hidden_states.shape[0], device=hidden_states.device,
                                        dtype=proj.dtype)
        else:
            self._validate_cache(cache, hidden_states.shape[0])
        mixed, next_cache = ops.step_projection(proj, self, cache, inplace=inplace)
        mixed = mixed.flatten(-2)
        if rows.shape[0] <= ops.DECODE_LINEAR_OUT_ROWS and ops.linear_supported(
                mixed, self.out_proj.weight) and (residual is None or residual.dtype == mixed.dtype):
            res = residual[:, 0] if residual is not None else None
            return ops.linear(mixed, self.out_proj.weight, res).unsqueeze(1), next_cache
        output = self.out_proj(mixed).unsqueeze(1)
        if residual is not None:
            output = residual + output
        return output, next_cache


class _Mamba3Block(nn.Module):
    def __init__(self, d_model: int, d_state: int, mimo_rank: int, causal: bool = True) -> None:
        super().__init__()
        self.norm = _RMSNorm(d_model)
        self.mixer = _Mamba3Mixer(d_model, d_state, mimo_rank, causal=causal)

    def forward(self, hidden_states, cache=None, *, return_cache: bool = False):
        mixed = self.mixer(self.norm(hidden_states), cache=cache, return_cache=return_cache)
        if return_cache:
            output, next_cache = mixed
            return hidden_states + output, next_cache
        return hidden_states + mixed

    def step(self, hidden_states, cache, *, inplace: bool = False):
        return self.mixer.step(hidden_states, cache, inplace=inplace, residual=hidden_states,
                               norm=self.norm)


class Mamba3(nn.Module):
    """A shape-preserving stack of Mamba-3 mixers (reference ``model.py:523-688``).

    ``Mamba3(d_model, d_state=128, depth=4, mimo_rank=1, causal=True)``; inputs and
    outputs are ``[batch, length, d_model]``.
    """

    def __init__(self, d_model: int, d_state: int = 128, depth: int = 4, mimo_rank: int = 1,
                 causal: bool = True) -> None:
        super().__init__()
        if d_model <= 0:
            raise ValueError("d_model must be positive")
        if d_state < 4:
            raise ValueError("d_state must be at least 4")
        if mimo_rank > 1 and d_state % 4 != 0:
            raise ValueError("MIMO requires d_state divisible by 4")
        if depth <= 0:
            raise ValueError("depth must be positive")
        if mimo_rank <= 0:
            raise ValueError("mimo_rank must be positive")
        self.d_model = d_model
        self.d_state = d_state
        self.depth = depth
        self.mimo_rank = mimo_rank
        self.causal = causal
        self.layers = nn.ModuleList(
            _Mamba3Block(d_model, d_state, mimo_rank, causal=causal) for _ in range(depth))
        self.norm_f = _RMSNorm(d_model)
        with torch.no_grad():
            for layer in self.layers:
                layer.mixer.out_proj.weight.div_(math.sqrt(depth))

    def _check_tokens(self, x: torch.Tensor, *, one_token: bool = False) -> None:
        """The input contract: ``[batch, length, d_model]``; length 1 for a decode step. The
        messages are the reference's (``model.py:570-579``), which callers match on."""
        shape = tuple(x.shape)
        if len(shape) != 3 or shape[2] != self.d_model:
            raise ValueError(f"expected [batch, length, {self.d_model}], got {shape}")
        if one_token and shape[1] != 1:
            raise ValueError(f"expected [batch, 1, {self.d_model}], got {shape}")

    def _norm_dtype(self, h: torch.Tensor) -> torch.dtype:
        """The dtype the next in_proj computes in: autocast's for FP32 rows, else the rows'."""
        if h.dtype == torch.float32 and torch.is_autocast_enabled(h.device.type):
            return torch.get_autocast_dtype(h.device.type)
        return h.dtype

    def _add_norm(self, h: torch.Tensor, mixed: torch.Tensor | None, norm: _RMSNorm,
                  out_dtype: torch.dtype, keep_sum: bool):
        """``(norm(h + mixed) as out_dtype, h + mixed)`` in one ``m3_rms_norm`` pass where it
        applies (ROCm rows, no autograd, a supported width), else the reference's ops."""
        sum_dtype = h.dtype if mixed is None else torch.promote_types(h.dtype, mixed.dtype)
        if sum_dtype == h.dtype and ops.rms_norm_supported(h, norm.weight, mixed, out_dtype):
            out, s = ops.rms_norm(h, norm.weight, norm.eps, add=mixed,
                                  keep_sum=keep_sum and mixed is not None, out_dtype=out_dtype)
            return out, (h if mixed is None else s)
        s = h if mixed is None else h + mixed
        return norm(s), s

    def _run_layers(self, x: torch.Tensor, *, return_cache: bool):
        """The layer loop of forward / prefill (reference ``model.py:585-607``): each block's
        residual add runs fused with the RMSNorm after it (the next block's, or norm_f)."""
        h, mixed, cache = x, None, []
        for layer in self.layers:
            normed, h = self._add_norm(h, mixed, layer.norm, self._norm_dtype(h), keep_sum=True)
            if return_cache:
                mixed, layer_cache = layer.mixer(normed, return_cache=True)
                cache.append(layer_cache)
            else:
                mixed = layer.mixer(normed)
        out, _ = self._add_norm(h, mixed, self.norm_f, h.dtype if mixed is None else
                                torch.promote_types(h.dtype, mixed.dtype), keep_sum=False)
        return out, cache

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        self._check_tokens(x)
        if x.numel() == 0:
            # no token to mix (batch or length 0): an empty result of the input's kind, with
            # no launch (this package computes no gradients, so nothing needs to depend on
            # the parameters)
            return torch.empty_like(x)
        return self._run_layers(x, return_cache=False)[0]

    def prefill(self, x: torch.Tensor):
        """Process a causal prefix and return the constant-size decode cache."""
        if not self.causal:
            raise ValueError("prefill requires causal=True")
        self._check_tokens(x)
        if x.numel() == 0:
            raise ValueError("prefill requires a non-empty batch and sequence")
        return self._run_layers(x, return_cache=True)

    def step(self, x: torch.Tensor, cache: list[_LayerCache] | None = None, *,
             inplace: bool = False):
        """Process one token while carrying the four recurrent states per layer.

        ``inplace=True`` updates the given cache tensors in place and returns them (used by
        the hipGraph decoder); the default leaves the given cache untouched.
        """
        if not self.causal:
            raise ValueError("step requires causal=True")
        self._check_tokens(x, one_token=True)
        depth = len(self.layers)
        if cache is not None and len(cache) != depth:
            raise ValueError(f"expected cache for {depth} layers")
        updated: list[_LayerCache] = []
        if x.shape[0] <= ops.DECODE_LINEAR_ROWS:
            # few rows: each block's RMSNorm and residual add run inside its two projections
            for i, layer in enumerate(self.layers):
                layer_cache = None if cache is None else cache[i]
                x, layer_cache = layer.step(x, layer_cache,
                                            inplace=inplace and layer_cache is not None)
                updated.append(layer_cache)
            return self.norm_f(x), updated
        # more rows (general GEMM projections): each residual add runs fused with the RMSNorm
        # after it, as in the forward's layer loop
        h, mixed = x, None
        for i, layer in enumerate(self.layers):
            layer_cache = None if cache is None else cache[i]
            normed, h = self._add_norm(h, mixed, layer.norm, self._norm_dtype(h), keep_sum=True)
            mixed, layer_cache = layer.mixer.step(normed, layer_cache,
                                                  inplace=inplace and layer_cache is not None)
            updated.append(layer_cache)
        out, _ = self._add_norm(h, mixed, self.norm_f, torch.promote_types(h.dtype, mixed.dtype),
                                keep_sum=False)
        return out, updated

    def set_chunk_sizes(self, *, training: int | None = None,
                        inference: int | None = None) -> Mamba3:
        """Set every mixer's chunk sizes. The HIP scan tiles the sequence itself; the chunk is
        validated, passed to the library as the caller's chunk, and used by the oracle."""
        sizes = {"training": training, "inference": inference}
        for name, size in sizes.items():
            if size is not None and size <= 0:
                raise ValueError(f"{name} chunk size must be positive")
        for layer in self.layers:
            mixer = layer.mixer
            mixer.chunk_size = mixer.chunk_size if training is None else training
            mixer.inference_chunk_size = (mixer.inference_chunk_size if inference is None
                                          else inference)
        return self

    def compile_layers(self, **kwargs: object) -> Mamba3:
        """Accepted for API compatibility; the HIP kernels are already fused."""
        return self

    def compile(self, **kwargs: object) -> Mamba3:  # type: ignore[override]
        """Accepted for API compatibility; returns this model unchanged."""
        return self

    def cuda_graph(self, batch_size: int = 1) -> _HipGraphDecoder:
        """Capture the complete stateful decode step in a hipGraph."""
        return _HipGraphDecoder(self, batch_size)


def _storage_signature(w: torch.Tensor) -> tuple[object, ...]:
    """What a captured graph depends on for one parameter: the same checks as the reference's
    ``_parameter_signature`` (``model.py:763-774``: identity, version, data pointer, device,
    dtype, shape), with the object itself kept instead of its ``id``."""
    return (w, w._version, w.data_ptr(), w.device, w.dtype, tuple(w.shape))


class _HipGraphDecoder:
    """A decode step of the whole stack, captured once in a hipGraph and replayed.

    The graph reads the static ``input`` buffer and updates the static per-layer ``cache``
    (``(phase, state, k_rot, value)``, the layer-cache layout) in place, so a replay is one
    input copy plus one graph launch. Decoding starts from zeros (``reset``) or from a
    prefill's cache (``load_cache``). The graph holds the addresses of the parameters it was
    captured with; ``validate`` refuses a model whose parameters were replaced or modified
    since. Interface of the reference's ``cuda_graph`` decoder (``model.py:691-774``).
    """

    def __init__(self, model: Mamba3, batch_size: int) -> None:
        if batch_size <= 0:
            raise ValueError("batch_size must be positive")
        weights = list(model.parameters())
        device, dtype = weights[0].device, weights[0].dtype
        if device.type != "cuda":
            raise ValueError("cuda_graph requires a ROCm (cuda) model")
        if model.training:
            raise ValueError("cuda_graph requires model.eval()")
        self.model = model
        # what the graph holds of each parameter: the object, its version counter, and the
        # storage it read (address, device, dtype, shape): `Module.to`, `.half()` or
        # `p.data = ...` keep the object and its version but move the storage
        self._captured = [_storage_signature(w) for w in weights]
        self.input = torch.zeros(batch_size, 1, model.d_model, device=device, dtype=dtype)
        self.cache = [layer.mixer.allocate_cache(batch_size, device=device, dtype=dtype)
                      for layer in model.layers]
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.device(device), torch.inference_mode():
            # One eager step first, on a side stream: the libraries' lazy set-up (handles,
            # workspaces, first-use allocations) must happen outside the capture.
            side = torch.cuda.Stream(device=device)
            side.wait_stream(torch.cuda.current_stream(device))
            with torch.cuda.stream(side):
                model.step(self.input, self.cache, inplace=True)
            torch.cuda.current_stream(device).wait_stream(side)
            with torch.cuda.graph(self.graph, stream=torch.cuda.Stream(device=device)):
                self.output, _ = model.step(self.input, self.cache, inplace=True)
        self.reset()

    def __call__(self, x: torch.Tensor, validate: bool = False) -> torch.Tensor:
        want = self.input
        if x.shape != want.shape:
            raise ValueError(f"expected {tuple(want.shape)}, got {tuple(x.shape)}")
        if (x.device, x.dtype) != (want.device, want.dtype):
            raise ValueError(f"expected {want.dtype} on {want.device}, "
                             f"got {x.dtype} on {x.device}")
        if x.requires_grad:
            raise ValueError("CUDA graph decoding does not support gradient inputs")
        if validate:
            self.validate()
        with torch.inference_mode(), torch.cuda.device(want.device):
            want.copy_(x)
            self.graph.replay()
        return self.output

    def replay(self) -> torch.Tensor:
        """Replay on whatever ``self.input`` holds (no copy, no checks)."""
        self.graph.replay()
        return self.output

    def validate(self) -> None:
        current = [_storage_signature(w) for w in self.model.parameters()]
        same = len(current) == len(self._captured) and all(
            now[0] is then[0] and now[1:] == then[1:]
            for now, then in zip(current, self._captured))
        if not same:
            raise RuntimeError("model state changed; recreate the CUDA graph decoder")

    def reset(self) -> None:
        """Start the next replay from an all-zero cache."""
        with torch.inference_mode():
            for layer_cache in self.cache:
                for t in layer_cache:
                    t.zero_()

    def load_cache(self, cache: list[_LayerCache]) -> None:
        """Continue decoding from ``cache`` (e.g. ``prefill``'s): copied into the static cache,
        whose tensors the graph holds."""
        if len(cache) != len(self.cache):
            raise ValueError(f"expected cache for {len(self.cache)} layers")
        with torch.inference_mode():
            for mine, given in zip(self.cache, cache):
                if len(given) != len(mine) or any(a.shape != b.shape
                                                  for a, b in zip(mine, given)):
                    raise ValueError(
                        f"expected cache shapes {tuple(tuple(t.shape) for t in mine)}, got "
                        f"{tuple(tuple(t.shape) for t in given)}")
                for a, b in zip(mine, given):
                    a.copy_(b)

"""WKV7 operators (MI355X-native), mirroring ``flashrwkv2.tmix.wkv7``.

Function names, keyword arguments, validation order and error types follow
the reference's ``flashrwkv2/tmix/wkv7/__init__.py`` (cited per function);
the native work goes through ``flashrwkv_amd._C`` into hand-written gfx950
HIP kernels. There is no CPU or Python fallback: without the native library
every operator raises RuntimeError.
"""

from __future__ import annotations

import torch

DECAY_LOGITS = 0
DECAY_RAW_W = 1


def _extension():
    """Native facade or RuntimeError (reference ``__init__.py:8-17``)."""
    import flashrwkv_amd

    extension = getattr(flashrwkv_amd, "_C", None)
    if extension is None:
        raise RuntimeError(
            "flashrwkv_amd native extension is not built; run "
            "`python -m flashrwkv_amd._build` before using the WKV7 operators"
        )
    return extension


def _validate_packed_inputs(*tensors: torch.Tensor) -> tuple[torch.Tensor, ...]:
    """Reference ``__init__.py:20-29``."""
    names = ("r", "decay_logits", "k", "v", "a", "b")
    for name, tensor in zip(names, tensors):
        if not isinstance(tensor, torch.Tensor):
            raise TypeError(f"{name} must be a torch.Tensor")
        if tensor.ndim != 3:
            raise ValueError(f"{name} must have packed shape [total_tokens,H,D]")
        if not tensor.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
    return tensors


def _validate_state(state: torch.Tensor) -> None:
    """Reference ``__init__.py:32-38``."""
    if not isinstance(state, torch.Tensor):
        raise TypeError("state_pool must be a torch.Tensor")
    if not state.is_contiguous():
        raise ValueError("state_pool must be contiguous")
    if state.dtype != torch.float32:
        raise TypeError("state_pool must have dtype float32")


def _validate_fp16_state(state: torch.Tensor) -> None:
    """Reference ``__init__.py:41-47``."""
    if not isinstance(state, torch.Tensor):
        raise TypeError("state_pool must be a torch.Tensor")
    if not state.is_contiguous():
        raise ValueError("state_pool must be contiguous")
    if state.dtype != torch.float16:
        raise TypeError("FP16-state state_pool must have dtype float16")


def _validate_fp16_elapsed_state(elapsed_state_pool: torch.Tensor,
                                 state_pool: torch.Tensor) -> None:
    """Reference ``__init__.py:50-62``."""
    if not isinstance(elapsed_state_pool, torch.Tensor):
        raise TypeError("elapsed_state_pool must be a torch.Tensor")
    if elapsed_state_pool.dtype != torch.int32:
        raise TypeError("elapsed_state_pool must have dtype torch.int32")
    if not elapsed_state_pool.is_cuda or not elapsed_state_pool.is_contiguous():
        raise ValueError("elapsed_state_pool must be contiguous CUDA int32")
    if elapsed_state_pool.device != state_pool.device:
        raise ValueError("elapsed_state_pool must share state_pool's device")
    if elapsed_state_pool.ndim != 1 or elapsed_state_pool.shape[0] != state_pool.shape[0]:
        raise ValueError("elapsed_state_pool must have shape [state_pool_slots]")


def _check_metadata_inputs(cu_seqlens: torch.Tensor, state_indices: torch.Tensor) -> None:
    """Reference ``__init__.py:154-163``."""
    if not isinstance(cu_seqlens, torch.Tensor):
        raise TypeError("cu_seqlens must be a torch.Tensor")
    if cu_seqlens.ndim != 1:
        raise ValueError("cu_seqlens must be one-dimensional")
    if not isinstance(state_indices, torch.Tensor):
        raise TypeError("state_indices must be a torch.Tensor")


def _resolve_max_seqlen(cu_seqlens: torch.Tensor, max_seqlen: int | None) -> int:
    """Reference ``__init__.py:166-177`` (synchronises when max_seqlen is None)."""
    if max_seqlen is not None:
        value = int(max_seqlen)
        if value <= 0:
            raise ValueError("max_seqlen must be positive")
        return value
    if cu_seqlens.numel() < 2:
        raise ValueError("cu_seqlens must contain at least one sequence")
    return int((cu_seqlens[1:] - cu_seqlens[:-1]).max().item())


def prepare_recurrent_metadata(
    cu_seqlens: torch.Tensor,
    state_indices: torch.Tensor,
    *,
    total_tokens: int,
    state_pool_size: int,
    max_seqlen: int | None = None,
) -> object:
    """Validate packed metadata and create a reusable native ticket.

    Reference ``__init__.py:180-197``. The ticket pins the metadata tensors
    (identity, data pointer, shape, version), launch sizes, device and the
    current stream; reusing it after any of these change raises RuntimeError.
    """
    _check_metadata_inputs(cu_seqlens, state_indices)
    return _extension().prepare_recurrent_metadata(
        cu_seqlens,
        state_indices,
        total_tokens,
        state_pool_size,
        -1 if max_seqlen is None else int(max_seqlen),
    )


def _run(r, decay, k, v, a, b, *, state, cu_seqlens, state_indices, scale,
         decay_bias, max_seqlen, validated_metadata, decay_mode=None):
    """Reference ``__init__.py:200-242``; ``decay_mode`` selects the internal op."""
    packed = _validate_packed_inputs(r, decay, k, v, a, b)
    _validate_state(state)
    _check_metadata_inputs(cu_seqlens, state_indices)
    ticket = (
        validated_metadata
        if validated_metadata is not None
        else prepare_recurrent_metadata(
            cu_seqlens,
            state_indices,
            total_tokens=r.shape[0],
            state_pool_size=state.shape[0],
            max_seqlen=max_seqlen,
        )
    )
    output = torch.empty_like(packed[3])
    extension = _extension()
    launch_max = -1 if max_seqlen is None else int(max_seqlen)
    if decay_mode is None:
        extension.recurrent_fp32_from_decay_logits(
            cu_seqlens, state_indices, state, *packed, output, float(scale),
            decay_bias, ticket, launch_max)
    else:
        extension.recurrent_fp32_forward_internal(
            cu_seqlens, state_indices, state, *packed, output, float(scale),
            int(decay_mode), decay_bias, ticket, launch_max)
    return output


def infer_recurrent_fp32io16_forward_varlen(
    r: torch.Tensor,
    decay_logits: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    a: torch.Tensor,
    b: torch.Tensor,
    *,
    state_pool: torch.Tensor,
    cu_seqlens: torch.Tensor,
    state_indices: torch.Tensor,
    scale: float = 1.0,
    decay_bias: torch.Tensor | None = None,
    max_seqlen: int | None = None,
    validated_metadata: object | None = None,
) -> torch.Tensor:
    """Run packed raw-decay RWKV-7 recurrence in-place on ``state_pool``.

    Reference ``__init__.py:245-277``: fp16/bf16 ``[N,H,D]`` tokens, fp32
    ``[slots,H,D,D]`` pool ([K,V]) updated at ``state_indices``; returns the
    output shaped like ``v``.
    """
    return _run(r, decay_logits, k, v, a, b, state=state_pool,
                cu_seqlens=cu_seqlens, state_indices=state_indices, scale=scale,
                decay_bias=decay_bias, max_seqlen=max_seqlen,
                validated_metadata=validated_metadata)


def recurrent_forward_internal(
    r: torch.Tensor,
    decay: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    a: torch.Tensor,
    b: torch.Tensor,
    *,
    state_pool: torch.Tensor,
    cu_seqlens: torch.Tensor,
    state_indices: torch.Tensor,
    decay_mode: int = DECAY_RAW_W,
    scale: float = 1.0,
    decay_bias: torch.Tensor | None = None,
    max_seqlen: int | None = None,
    validated_metadata: object | None = None,
) -> torch.Tensor:
    """Internal fp32-state recurrent op with an explicit decay mode.

    Not part of the reference API: ``decay_mode=DECAY_RAW_W`` takes the
    retention ``w`` itself (needed for inputs below the logits floor
    ``exp(-e^{-1/2})``) and fp32 tokens are accepted (the public op rejects
    them, reference ``csrc/validation.cpp:100-103``).
    """
    return _run(r, decay, k, v, a, b, state=state_pool, cu_seqlens=cu_seqlens,
                state_indices=state_indices, scale=scale, decay_bias=decay_bias,
                max_seqlen=max_seqlen, validated_metadata=validated_metadata,
                decay_mode=decay_mode)


def infer_recurrent_fp16_advance_i32(elapsed_state: torch.Tensor, amount: int) -> None:
    """Advance the fp16-state elapsed/dither phase origins in place.

    Reference ``__init__.py:65-81``.
    """
    if not isinstance(elapsed_state, torch.Tensor):
        raise TypeError("elapsed_state must be a torch.Tensor")
    if elapsed_state.dtype != torch.int32:
        raise TypeError("elapsed_state must have dtype torch.int32")
    if not elapsed_state.is_cuda or not elapsed_state.is_contiguous():
        raise ValueError("elapsed_state must be contiguous CUDA int32")
    if elapsed_state.numel() == 0:
        raise ValueError("elapsed_state must be non-empty")
    if not isinstance(amount, int) or isinstance(amount, bool):
        raise TypeError("amount must be an int")
    _extension().recurrent_fp16_advance_i32(elapsed_state, amount)


def infer_recurrent_fp16_advance_i32_varlen(
    elapsed_state_pool: torch.Tensor,
    cu_seqlens: torch.Tensor,
    state_indices: torch.Tensor,
    *,
    total_tokens: int,
    validated_metadata: object | None = None,
) -> None:
    """Advance the selected slots' phase origins by their packed lengths.

    Reference ``__init__.py:83-130``.
    """
    if not isinstance(elapsed_state_pool, torch.Tensor):
        raise TypeError("elapsed_state_pool must be a torch.Tensor")
    if (
        elapsed_state_pool.dtype != torch.int32
        or not elapsed_state_pool.is_cuda
        or not elapsed_state_pool.is_contiguous()
        or elapsed_state_pool.ndim != 1
        or elapsed_state_pool.numel() == 0
    ):
        raise ValueError("elapsed_state_pool must be non-empty contiguous CUDA int32")
    _check_metadata_inputs(cu_seqlens, state_indices)
    if cu_seqlens.dtype != torch.int32 or not cu_seqlens.is_cuda or not cu_seqlens.is_contiguous():
        raise ValueError("cu_seqlens must be contiguous CUDA int32")
    if (state_indices.dtype != torch.int32 or not state_indices.is_cuda
            or not state_indices.is_contiguous()):
        raise ValueError("state_indices must be contiguous CUDA int32")
    if (cu_seqlens.device != elapsed_state_pool.device
            or state_indices.device != elapsed_state_pool.device):
        raise ValueError("elapsed metadata tensors must share a CUDA device")
    if (cu_seqlens.ndim != 1 or state_indices.ndim != 1
            or cu_seqlens.numel() != state_indices.numel() + 1):
        raise ValueError("cu_seqlens must have shape [B+1] and state_indices shape [B]")
    if not isinstance(total_tokens, int) or isinstance(total_tokens, bool) or total_tokens <= 0:
        raise ValueError("total_tokens must be a positive integer")
    ticket = (
        validated_metadata
        if validated_metadata is not None
        else prepare_recurrent_metadata(
            cu_seqlens,
            state_indices,
            total_tokens=total_tokens,
            state_pool_size=elapsed_state_pool.shape[0],
        )
    )
    _extension().recurrent_fp16_advance_i32_varlen(
        cu_seqlens, state_indices, elapsed_state_pool, total_tokens, ticket)


def infer_recurrent_add_vec_forward_varlen(x: torch.Tensor, vec: torch.Tensor) -> torch.Tensor:
    """``fp16(x + vec)`` over packed ``[N,C]`` rows (reference ``__init__.py:133-151``)."""
    for name, tensor in (("x", x), ("vec", vec)):
        if not isinstance(tensor, torch.Tensor):
            raise TypeError(f"{name} must be a torch.Tensor")
        if tensor.dtype != torch.float16:
            raise TypeError(f"{name} must have dtype torch.float16")
        if not tensor.is_cuda or not tensor.is_contiguous():
            raise ValueError(f"{name} must be contiguous CUDA float16")
        if tensor.device != x.device:
            raise ValueError(f"{name} must share x's device")
    if x.ndim != 2 or x.shape[0] <= 0 or x.shape[1] <= 0 or x.shape[1] % 2:
        raise ValueError("x must have packed shape [total_tokens,C] with even C")
    if vec.shape != (x.shape[1],):
        raise ValueError("vec must have shape [C]")
    return _extension().recurrent_add_vec_forward_varlen(x, vec)


def infer_recurrent_fp16_forward_varlen(
    r: torch.Tensor,
    decay_logits: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    a: torch.Tensor,
    b: torch.Tensor,
    *,
    state_pool: torch.Tensor,
    elapsed_state_pool: torch.Tensor,
    cu_seqlens: torch.Tensor,
    state_indices: torch.Tensor,
    scale: float = 1.0,
    decay_bias: torch.Tensor | None = None,
    max_seqlen: int | None = None,
    validated_metadata: object | None = None,
) -> torch.Tensor:
    """Packed recurrence with an fp16 state pool (the Albatross family).

    Reference ``__init__.py:280-339``: fp16 ``[N,H,D]`` tokens and decay
    logits, fp16 ``[slots,H,D,D]`` pool ([K,V]) updated at ``state_indices``,
    int32 ``elapsed_state_pool`` phase origins (read, not advanced); returns
    the fp16 output shaped like ``v``.
    """
    packed = _validate_packed_inputs(r, decay_logits, k, v, a, b)
    _validate_fp16_state(state_pool)
    _validate_fp16_elapsed_state(elapsed_state_pool, state_pool)
    _check_metadata_inputs(cu_seqlens, state_indices)
    if max_seqlen is None:
        # The ticket infers it; no host read of the offsets per launch.
        launch_max_seqlen = -1
    else:
        if not isinstance(max_seqlen, int) or isinstance(max_seqlen, bool) or max_seqlen <= 0:
            raise ValueError("max_seqlen must be a positive integer")
        launch_max_seqlen = int(max_seqlen)
    ticket = (
        validated_metadata
        if validated_metadata is not None
        else prepare_recurrent_metadata(
            cu_seqlens,
            state_indices,
            total_tokens=r.shape[0],
            state_pool_size=state_pool.shape[0],
            max_seqlen=None if launch_max_seqlen < 0 else launch_max_seqlen,
        )
    )
    output = torch.empty_like(packed[3])
    _extension().recurrent_fp16_from_decay_logits(
        cu_seqlens, state_indices, elapsed_state_pool, state_pool, *packed, output,
        float(scale), decay_bias, ticket, launch_max_seqlen)
    return output


__all__ = [
    "infer_recurrent_fp16_advance_i32",
    "infer_recurrent_fp16_advance_i32_varlen",
    "infer_recurrent_add_vec_forward_varlen",
    "infer_recurrent_fp32io16_forward_varlen",
    "infer_recurrent_fp16_forward_varlen",
    "prepare_recurrent_metadata",
]

# Reference ``tmix/wkv7/__init__.py:350-354`` re-exports the pretraining and
# chunk entries here.
from .pretrain import pretrain_recurrent_bf16  # noqa: E402
from .chunk import infer_chunk_bf16_forward_varlen  # noqa: E402

__all__.extend(["pretrain_recurrent_bf16", "infer_chunk_bf16_forward_varlen"])

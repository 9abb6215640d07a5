"""ctypes binding of the C ABI in ``include/flashrwkv_amd.h``.

This is the binding a non-torch host (or a test of the boundary itself) uses:
every call passes raw device pointers, sizes and the current HIP stream to
``libflashrwkv_amd.so`` and turns a non-zero status into RuntimeError with
``frwkv_last_error()``. Tensors are only a convenient way to own device
memory here; the library never sees a torch type.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch

LIBRARY = Path(__file__).resolve().parent / "libflashrwkv_amd.so"

DTYPE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}
DECAY_LOGITS, DECAY_RAW_W = 0, 1

_INT, _I32, _I64 = ctypes.c_int, ctypes.c_int32, ctypes.c_int64
_F32, _VP, _SZ = ctypes.c_float, ctypes.c_void_p, ctypes.c_size_t

# name -> argtypes, in the header's parameter order.
SIGNATURES = {
    "frwkv_abi_version": [],
    "frwkv_status_string": [_INT],
    "frwkv_last_error": [],
    "frwkv_metadata_validate": [_VP, _VP, _I32, _I32, _I32, _VP, _VP, _VP, _VP],
    "frwkv_recurrent_forward": [_INT, _INT] + [_I32] * 6 + [_VP] * 12 + [_F32, _VP],
    "frwkv_chunk_forward": [_INT] * 3 + [_I32] * 5 + [_VP] * 12 + [_F32, _VP],
    "frwkv_statetune_forward": [_INT] * 2 + [_I32] * 5 + [_VP] * 15 + [_F32, _VP],
    "frwkv_statetune_interior_bytes": [_I32] * 3,
    "frwkv_statetune_interior": [_INT] * 2 + [_I32] * 4 + [_VP] * 11 + [_VP],
    "frwkv_statetune_backward": [_INT] * 2 + [_I32] * 5 + [_VP] * 22 + [_SZ, _F32, _VP],
    "frwkv_statetune_backward_workspace_bytes": [_I32] * 3 + [_INT],
    "frwkv_statetune_backward_noalloc": [_INT] * 2 + [_I32] * 5 + [_VP] * 21 + [_F32, _VP],
    "frwkv_pretrain_forward": [_INT] * 2 + [_I32] * 4 + [_VP] * 10,
    "frwkv_pretrain_backward": [_INT] * 2 + [_I32] * 4 + [_VP] * 15 + [_SZ, _VP],
    "frwkv_pretrain_backward_workspace_bytes": [_I32] * 4,
    "frwkv_chunk_replay": [_INT] * 2 + [_I32] * 4 + [_VP] * 12 + [_F32, _VP],
    "frwkv_recurrent_fp16_forward": [_I32] * 6 + [_VP] * 13 + [_F32, _VP],
    "frwkv_advance_i32": [_VP, _I64, _I32, _VP],
    "frwkv_advance_i32_varlen": [_I32] * 2 + [_VP] * 5,
    "frwkv_add_vec": [_I64, _I32] + [_VP] * 4,
    "frwkv_kk_a_gate": [_INT, _I64, _I32, _I32] + [_VP] * 9,
    "frwkv_lnx_rkvres_xg": [_INT, _I64, _I32, _I32] + [_VP] * 10,
    "frwkv_lnx_pretrain_forward": [_INT, _I64, _I32, _I32] + [_VP] * 12,
    "frwkv_lnx_pretrain_backward_workspace_bytes": [_I64, _I32, _I32],
    "frwkv_lnx_pretrain_backward": [_INT, _I64, _I32, _I32] + [_VP] * 20 + [_SZ, _VP],
    "frwkv_recurrent_tmix_fused_forward": [_INT] * 2 + [_I32] * 5 + [_VP] * 18 + [_F32, _VP],
}

_LIB = None


def library() -> ctypes.CDLL:
    """The loaded ``libflashrwkv_amd.so`` (ImportError if it is not built)."""
    global _LIB
    if _LIB is None:
        if not LIBRARY.exists():
            raise ImportError(f"{LIBRARY.name} is not built; run `python -m flashrwkv_amd._build`")
        lib = ctypes.CDLL(str(LIBRARY))
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = ctypes.c_size_t if name.endswith("_bytes") else ctypes.c_int
        lib.frwkv_status_string.restype = ctypes.c_char_p
        lib.frwkv_last_error.restype = ctypes.c_char_p
        _LIB = lib
    return _LIB


def _p(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _check(status: int) -> None:
    if status != 0:
        lib = library()
        raise RuntimeError(f"{lib.frwkv_status_string(status).decode()}: "
                           f"{lib.frwkv_last_error().decode()}")


def metadata_validate(cu_seqlens, state_indices, total_tokens, state_pool_size):
    """Device validation + snapshot; returns ``(status, cu_snapshot, slot_snapshot)``."""
    status = torch.empty(1, dtype=torch.int32, device=cu_seqlens.device)
    cu_snap = torch.empty_like(cu_seqlens)
    slot_snap = torch.empty_like(state_indices)
    _check(library().frwkv_metadata_validate(
        _p(cu_seqlens), _p(state_indices), state_indices.numel(), int(total_tokens),
        int(state_pool_size), _p(status), _p(cu_snap), _p(slot_snap), _stream()))
    return status, cu_snap, slot_snap


def recurrent_forward(r, decay, k, v, a, b, *, state_pool, cu_seqlens, state_indices,
                      metadata_status, output, scale=1.0, decay_mode=DECAY_RAW_W,
                      decay_bias=None, max_seqlen=-1):
    n, h, d = r.shape
    _check(library().frwkv_recurrent_forward(
        DTYPE[r.dtype], decay_mode, state_indices.numel(), h, d, n, int(max_seqlen),
        state_pool.shape[0], _p(cu_seqlens), _p(state_indices), _p(metadata_status),
        _p(state_pool), _p(r), _p(decay), _p(decay_bias), _p(k), _p(v), _p(a), _p(b),
        _p(output), float(scale), _stream()))


def chunk_forward(r, decay, k, v, a, b, *, state_pool, cu_seqlens, state_indices,
                  metadata_status, output, scale=1.0, decay_mode=DECAY_RAW_W,
                  decay_bias=None):
    n, h, d = r.shape
    _check(library().frwkv_chunk_forward(
        DTYPE[r.dtype], decay_mode, DTYPE[state_pool.dtype], state_indices.numel(), h, d,
        n, state_pool.shape[0], _p(cu_seqlens), _p(state_indices), _p(metadata_status),
        _p(state_pool), _p(r), _p(decay), _p(decay_bias), _p(k), _p(v), _p(a), _p(b),
        _p(output), float(scale), _stream()))


def statetune_forward(r, decay, k, v, a, b, *, sequence_chunk_offsets, chunk_token_starts,
                      chunk_token_ends, state, output, boundary, state_dot_a, interior=None,
                      scale=1.0, decay_mode=DECAY_RAW_W, decay_bias=None):
    n, h, d = r.shape
    _check(library().frwkv_statetune_forward(
        DTYPE[r.dtype], decay_mode, sequence_chunk_offsets.numel() - 1, h, d, n,
        chunk_token_starts.numel(), _p(sequence_chunk_offsets), _p(chunk_token_starts),
        _p(chunk_token_ends), _p(state), _p(r), _p(decay), _p(decay_bias), _p(k), _p(v),
        _p(a), _p(b), _p(output), _p(boundary), _p(state_dot_a), _p(interior), float(scale),
        _stream()))


def statetune_interior_bytes(head_size: int, heads: int, total_tokens: int) -> int:
    return int(library().frwkv_statetune_interior_bytes(head_size, heads, total_tokens))


def statetune_backward_workspace_bytes(head_size: int, heads: int, total_tokens: int,
                                       interior_given: bool) -> int:
    return int(library().frwkv_statetune_backward_workspace_bytes(
        head_size, heads, total_tokens, int(bool(interior_given))))


def workspace(nbytes: int, device) -> torch.Tensor | None:
    """Device scratch of ``nbytes`` (None for 0)."""
    return None if nbytes == 0 else torch.empty(nbytes, dtype=torch.uint8, device=device)


def statetune_backward(r, decay, k, v, a, b, *, sequence_chunk_offsets, chunk_token_starts,
                       chunk_token_ends, boundary, grad_output, grad_final_state, grads,
                       grad_initial_state, interior=None, work=None, scale=1.0,
                       decay_mode=DECAY_RAW_W, decay_bias=None):
    """``grads`` = (grad_r, grad_decay, grad_k, grad_v, grad_a, grad_b). ``work``:
    the workspace (allocated here when None and needed)."""
    n, h, d = r.shape
    if work is None:
        work = workspace(statetune_backward_workspace_bytes(d, h, n, interior is not None),
                         r.device)
    _check(library().frwkv_statetune_backward(
        DTYPE[r.dtype], decay_mode, sequence_chunk_offsets.numel() - 1, h, d, n,
        chunk_token_starts.numel(), _p(sequence_chunk_offsets), _p(chunk_token_starts),
        _p(chunk_token_ends), _p(boundary), _p(interior), _p(r), _p(decay), _p(decay_bias),
        _p(k), _p(v), _p(a), _p(b), _p(grad_output), _p(grad_final_state),
        *(_p(g) for g in grads), _p(grad_initial_state), _p(work),
        0 if work is None else work.numel(), float(scale), _stream()))


NOALLOC_SCRATCH_BYTES = 64 << 20  # FRWKV_NOALLOC_SCRATCH_BYTES


def statetune_backward_noalloc(r, decay, k, v, a, b, *, sequence_chunk_offsets,
                               chunk_token_starts, chunk_token_ends, boundary, grad_output,
                               grad_final_state, grads, grad_initial_state, interior=None,
                               scale=1.0, decay_mode=DECAY_RAW_W, decay_bias=None):
    """frwkv_statetune_backward_noalloc: the workspace is the library's static
    per-device scratch; nothing is allocated."""
    n, h, d = r.shape
    _check(library().frwkv_statetune_backward_noalloc(
        DTYPE[r.dtype], decay_mode, sequence_chunk_offsets.numel() - 1, h, d, n,
        chunk_token_starts.numel(), _p(sequence_chunk_offsets), _p(chunk_token_starts),
        _p(chunk_token_ends), _p(boundary), _p(interior), _p(r), _p(decay), _p(decay_bias),
        _p(k), _p(v), _p(a), _p(b), _p(grad_output), _p(grad_final_state),
        *(_p(g) for g in grads), _p(grad_initial_state), float(scale), _stream()))


def pretrain_forward(r, decay, k, v, a, b, *, output, boundary, state_dot_a,
                     decay_mode=DECAY_LOGITS):
    """Dense [B,T,H,D] tokens; boundary [B,H,T/16,D,D]; state_dot_a [B,T,H,D]."""
    bsz, t_len, h, d = r.shape
    _check(library().frwkv_pretrain_forward(
        DTYPE[r.dtype], decay_mode, bsz, t_len, h, d, _p(r), _p(decay), _p(k), _p(v), _p(a),
        _p(b), _p(output), _p(boundary), _p(state_dot_a), _stream()))


def pretrain_backward(r, decay, k, v, a, b, *, grad_output, boundary, grads,
                      decay_mode=DECAY_LOGITS):
    """``grads`` = (grad_r, grad_decay, grad_k, grad_v, grad_a, grad_b)."""
    bsz, t_len, h, d = r.shape
    work = workspace(int(library().frwkv_pretrain_backward_workspace_bytes(bsz, t_len, h, d)),
                     r.device)
    _check(library().frwkv_pretrain_backward(
        DTYPE[r.dtype], decay_mode, bsz, t_len, h, d, _p(r), _p(decay), _p(k), _p(v), _p(a),
        _p(b), _p(grad_output), _p(boundary), *(_p(g) for g in grads), _p(work),
        0 if work is None else work.numel(), _stream()))


def chunk_replay(r, decay, k, v, a, b, *, chunk_token_starts, chunk_token_ends, boundary,
                 output, state_dot_a, scale=1.0, decay_mode=DECAY_LOGITS, decay_bias=None):
    """RL/infctx replay stage: every chunk from its boundary state."""
    n, h, d = r.shape
    _check(library().frwkv_chunk_replay(
        DTYPE[r.dtype], decay_mode, chunk_token_starts.numel(), h, d, n,
        _p(chunk_token_starts), _p(chunk_token_ends), _p(boundary), _p(r), _p(decay),
        _p(decay_bias), _p(k), _p(v), _p(a), _p(b), _p(output), _p(state_dot_a),
        float(scale), _stream()))


def recurrent_fp16_forward(r, decay_logits, k, v, a, b, *, state_pool, elapsed_state_pool,
                           cu_seqlens, state_indices, metadata_status, output, scale=1.0,
                           decay_bias=None, max_seqlen=-1):
    """fp16-state family: fp16 tokens and pool, int32 phase origins (read only)."""
    n, h, d = r.shape
    _check(library().frwkv_recurrent_fp16_forward(
        state_indices.numel(), h, d, n, int(max_seqlen), state_pool.shape[0], _p(cu_seqlens),
        _p(state_indices), _p(metadata_status), _p(elapsed_state_pool), _p(state_pool), _p(r),
        _p(decay_logits), _p(decay_bias), _p(k), _p(v), _p(a), _p(b), _p(output),
        float(scale), _stream()))


def advance_i32(elapsed_state, amount):
    _check(library().frwkv_advance_i32(_p(elapsed_state), elapsed_state.numel(), int(amount),
                                       _stream()))


def advance_i32_varlen(elapsed_state_pool, *, cu_seqlens, state_indices, metadata_status):
    _check(library().frwkv_advance_i32_varlen(
        state_indices.numel(), elapsed_state_pool.numel(), _p(cu_seqlens), _p(state_indices),
        _p(metadata_status), _p(elapsed_state_pool), _stream()))


def add_vec(x, vec, output):
    rows, channels = x.shape
    _check(library().frwkv_add_vec(rows, channels, _p(x), _p(vec), _p(output), _stream()))


def kk_a_gate(k, k_k, a0, a12, k_a, *, new_k, neg_kk, kka, head_size=64):
    """TMix producer on packed ``[N, C]`` rows (C = H * head_size)."""
    n, c = k.shape
    _check(library().frwkv_kk_a_gate(
        DTYPE[k.dtype], n, c // head_size, head_size, _p(k), _p(k_k), _p(a0), _p(a12),
        _p(k_a), _p(new_k), _p(neg_kk), _p(kka), _stream()))


def lnx_rkvres_xg(x, r, k, v, r_k, weight, bias, g, *, output, head_size=64):
    """TMix consumer on packed ``[N, C]`` rows (C = H * head_size)."""
    n, c = x.shape
    _check(library().frwkv_lnx_rkvres_xg(
        DTYPE[x.dtype], n, c // head_size, head_size, _p(x), _p(r), _p(k), _p(v), _p(r_k),
        _p(weight), _p(bias), _p(g), _p(output), _stream()))


def recurrent_tmix_fused_forward(r, decay, k, v, a12, g, k_k, a0, k_a, r_k, ln_weight,
                                 ln_bias, *, state_pool, cu_seqlens, state_indices,
                                 metadata_status, output, scale=1.0, decay_mode=DECAY_LOGITS,
                                 decay_bias=None):
    """Fused kk_a_gate -> WKV7 -> lnx_rkvres_xg (head size 64, fp32 pool)."""
    n, h, d = r.shape
    _check(library().frwkv_recurrent_tmix_fused_forward(
        DTYPE[r.dtype], decay_mode, state_indices.numel(), h, d, n, state_pool.shape[0],
        _p(cu_seqlens), _p(state_indices), _p(metadata_status), _p(state_pool), _p(r),
        _p(decay), _p(decay_bias), _p(k), _p(v), _p(a12), _p(g), _p(k_k), _p(a0), _p(k_a),
        _p(r_k), _p(ln_weight), _p(ln_bias), _p(output), float(scale), _stream()))


def lnx_pretrain_forward(x, r, k, v, residual_scale, weight, bias, g, *, output, mean, rstd,
                         head_size=64):
    """Training consumer forward over ``[N, C]`` (or ``[B, T, C]``) tokens;
    ``mean`` / ``rstd`` fp32 with N * C / head_size elements."""
    c = x.shape[-1]
    n = x.numel() // c
    _check(library().frwkv_lnx_pretrain_forward(
        DTYPE[x.dtype], n, c // head_size, head_size, _p(x), _p(r), _p(k), _p(v),
        _p(residual_scale), _p(weight), _p(bias), _p(g), _p(output), _p(mean), _p(rstd),
        _stream()))


def lnx_pretrain_backward(grad_output, x, r, k, v, residual_scale, weight, bias, g, mean,
                          rstd, *, grads, head_size=64, work=None):
    """``grads`` = (grad_x, grad_r, grad_k, grad_v, grad_residual_scale,
    grad_weight, grad_bias, grad_g)."""
    c = x.shape[-1]
    n = x.numel() // c
    need = int(library().frwkv_lnx_pretrain_backward_workspace_bytes(n, c // head_size,
                                                                      head_size))
    if work is None:
        work = workspace(need, x.device)
    _check(library().frwkv_lnx_pretrain_backward(
        DTYPE[x.dtype], n, c // head_size, head_size, _p(grad_output), _p(x), _p(r), _p(k),
        _p(v), _p(residual_scale), _p(weight), _p(bias), _p(g), _p(mean), _p(rstd),
        *(_p(t) for t in grads), _p(work), 0 if work is None else work.numel(), _stream()))

"""Native extension facade (the counterpart of the reference's ``flashrwkv2._C``).

Loads ``_flashrwkv_amd_ops.so`` (the TORCH_LIBRARY binding over
``libflashrwkv_amd.so``) and exposes the reference's native callable names
with the reference's positional argument order, so code written against
``flashrwkv2._C`` (e.g. reference tests calling
``_C.recurrent_fp32_from_decay_logits`` directly) runs unchanged.

Importing this module raises ImportError when the native libraries are not
built; there is no Python or CPU fallback.
"""

from __future__ import annotations

from pathlib import Path

import torch

_PKG = Path(__file__).resolve().parent
OPS_LIBRARY = _PKG / "_flashrwkv_amd_ops.so"
HIP_LIBRARY = _PKG / "libflashrwkv_amd.so"

if not OPS_LIBRARY.exists() or not HIP_LIBRARY.exists():
    raise ImportError(
        "flashrwkv_amd native libraries are not built "
        f"({OPS_LIBRARY.name}, {HIP_LIBRARY.name}); run "
        "`python -m flashrwkv_amd._build`"
    )

torch.ops.load_library(str(OPS_LIBRARY))
ops = torch.ops.flashrwkv2
# The same library is also a Python extension module: direct (pybind11)
# entry points for the per-token decode chain, which run the same C++
# functions as the ops above without the dispatcher's boxed call.
from . import _flashrwkv_amd_ops as direct  # noqa: E402


def prepare_recurrent_metadata(query_start_loc, state_indices, total_tokens,
                               state_pool_size, max_seqlen=-1):
    return ops.prepare_recurrent_metadata(
        query_start_loc, state_indices, int(total_tokens), int(state_pool_size),
        int(max_seqlen))


def recurrent_fp32_from_decay_logits(query_start_loc, state_indices, state, r,
                                     decay_logits, k, v, a, b, output, scale,
                                     decay_bias=None, validated_metadata=None,
                                     max_seqlen=-1):
    direct.recurrent_fp32_from_decay_logits(
        query_start_loc, state_indices, state, r, decay_logits, k, v, a, b,
        output, float(scale), decay_bias, validated_metadata, int(max_seqlen))


def recurrent_fp32_forward_internal(query_start_loc, state_indices, state, r,
                                    decay, k, v, a, b, output, scale, decay_mode,
                                    decay_bias=None, validated_metadata=None,
                                    max_seqlen=-1):
    direct.recurrent_fp32_forward_internal(
        query_start_loc, state_indices, state, r, decay, k, v, a, b, output,
        float(scale), int(decay_mode), decay_bias, validated_metadata,
        int(max_seqlen))


def set_recurrent_long_route(route):
    """Route of long bf16 sequences in the fp32-state op (0 split-precision
    chunk kernel, 1 per-token fp32 kernel); returns the previous route."""
    return int(ops.set_recurrent_long_route(int(route)))


def recurrent_long_route():
    return int(ops.recurrent_long_route())


def loaded_libraries() -> list[str]:
    """Absolute paths of the native libraries this facade loaded."""
    return [str(HIP_LIBRARY), str(OPS_LIBRARY)]


def infer_chunk_bf16_forward_varlen(r, decay_logits, k, v, a, b, state_pool, cu_seqlens,
                                    state_indices, chunk_size=16, max_seqlen=-1,
                                    scale=1.0, decay_bias=None):
    return ops.infer_chunk_bf16_forward_varlen(
        r, decay_logits, k, v, a, b, state_pool, cu_seqlens, state_indices,
        int(chunk_size), int(max_seqlen), float(scale), decay_bias)


def chunk_forward_internal(r, decay, k, v, a, b, state_pool, cu_seqlens, state_indices,
                           scale, decay_mode, decay_bias=None):
    return ops.chunk_forward_internal(r, decay, k, v, a, b, state_pool, cu_seqlens,
                                      state_indices, float(scale), int(decay_mode),
                                      decay_bias)


def statetune_recurrent_fp32io16_forward(sequence_chunk_offsets, chunk_token_starts,
                                         chunk_token_ends, state, r, decay_logits, k, v,
                                         a, b, output, boundary, state_dot_a, scale=1.0):
    ops.statetune_recurrent_fp32io16_forward(
        sequence_chunk_offsets, chunk_token_starts, chunk_token_ends, state, r,
        decay_logits, k, v, a, b, output, boundary, state_dot_a, float(scale))


def statetune_forward_internal(sequence_chunk_offsets, chunk_token_starts,
                               chunk_token_ends, state, r, decay, k, v, a, b, output,
                               boundary, state_dot_a, interior, scale, decay_mode):
    ops.statetune_forward_internal(
        sequence_chunk_offsets, chunk_token_starts, chunk_token_ends, state, r, decay,
        k, v, a, b, output, boundary, state_dot_a, interior, float(scale), int(decay_mode))


def statetune_recurrent_fp32io16_backward(sequence_chunk_offsets, chunk_token_starts,
                                          chunk_token_ends, final_state, r, decay_logits, k,
                                          v, a, b, state_dot_a, grad_output, grad_final_state,
                                          boundary, grad_r, grad_decay_logits, grad_k, grad_v,
                                          grad_a, grad_b, grad_initial_state, scale=1.0):
    ops.statetune_recurrent_fp32io16_backward(
        sequence_chunk_offsets, chunk_token_starts, chunk_token_ends, final_state, r,
        decay_logits, k, v, a, b, state_dot_a, grad_output, grad_final_state, boundary,
        grad_r, grad_decay_logits, grad_k, grad_v, grad_a, grad_b, grad_initial_state,
        float(scale))


def statetune_backward_internal(sequence_chunk_offsets, chunk_token_starts, chunk_token_ends,
                                r, decay, k, v, a, b, grad_output, grad_final_state, boundary,
                                grad_r, grad_decay, grad_k, grad_v, grad_a, grad_b,
                                grad_initial_state, interior, scale, decay_mode):
    ops.statetune_backward_internal(
        sequence_chunk_offsets, chunk_token_starts, chunk_token_ends, r, decay, k, v, a, b,
        grad_output, grad_final_state, boundary, grad_r, grad_decay, grad_k, grad_v, grad_a,
        grad_b, grad_initial_state, interior, float(scale), int(decay_mode))


def rl_infctx_chunk_fp32io16_forward(sequence_chunk_offsets, chunk_token_starts,
                                     chunk_token_ends, state, r, decay_logits, k, v, a, b,
                                     strategy=1, scale=1.0, decay_bias=None):
    """Reference rl_infctx_chunk_fp32io16_forward.cpp:157-241: returns (output, working_state)."""
    return ops.rl_infctx_chunk_fp32io16_forward(
        sequence_chunk_offsets, chunk_token_starts, chunk_token_ends, state, r, decay_logits,
        k, v, a, b, int(strategy), float(scale), decay_bias)


def rl_infctx_chunk_fp32io16_backward_replay(chunk_token_starts, chunk_token_ends, boundary, r,
                                             decay_logits, k, v, a, b, output, state_dot_a,
                                             scale=1.0, decay_bias=None):
    """Reference rl_infctx_chunk_fp32io16_backward.cpp:102-135."""
    ops.rl_infctx_chunk_fp32io16_backward_replay(
        chunk_token_starts, chunk_token_ends, boundary, r, decay_logits, k, v, a, b, output,
        state_dot_a, float(scale), decay_bias)


def recurrent_fp16_from_decay_logits(query_start_loc, state_indices, elapsed_state_pool, state,
                                     r, decay_logits, k, v, a, b, output, scale,
                                     decay_bias=None, validated_metadata=None, max_seqlen=-1):
    """Reference infer_recurrent_fp16_forward_varlen.cpp:210-270, 289-301."""
    direct.recurrent_fp16_from_decay_logits(
        query_start_loc, state_indices, elapsed_state_pool, state, r, decay_logits, k, v, a,
        b, output, float(scale), decay_bias, validated_metadata, int(max_seqlen))


def recurrent_fp16_advance_i32(elapsed_state, amount):
    """Reference infer_recurrent_fp16_forward_varlen.cpp:129-135."""
    direct.recurrent_fp16_advance_i32(elapsed_state, int(amount))


def recurrent_fp16_advance_i32_varlen(query_start_loc, state_indices, elapsed_state_pool,
                                      total_tokens, validated_metadata=None):
    """Reference infer_recurrent_fp16_forward_varlen.cpp:137-191."""
    direct.recurrent_fp16_advance_i32_varlen(query_start_loc, state_indices,
                                             elapsed_state_pool, int(total_tokens),
                                             validated_metadata)


def recurrent_add_vec_forward_varlen(x, vec):
    """Reference infer_recurrent_fp16_forward_varlen.cpp:193-208."""
    return direct.recurrent_add_vec_forward_varlen(x, vec)


def tmix_kk_a_gate_forward_varlen(k, k_k, a0, a12, k_a, head_size=64, batch_size=1,
                                  max_seqlen=1):
    """Reference kk_a_gate/infer_fp16_forward_varlen.cpp:41-85: returns (new_k, neg_kk, kka)."""
    return direct.tmix_kk_a_gate_forward_varlen(k, k_k, a0, a12, k_a, int(head_size),
                                                int(batch_size), int(max_seqlen))


def tmix_lnx_rkvres_xg_forward_varlen(x, r, k, v, r_k, weight, bias, g, head_size=64,
                                      batch_size=1, max_seqlen=1):
    """Reference lnx_rkvres_xg/infer_fp16_forward_varlen.cpp:40-98."""
    return direct.tmix_lnx_rkvres_xg_forward_varlen(x, r, k, v, r_k, weight, bias, g,
                                                    int(head_size), int(batch_size),
                                                    int(max_seqlen))


def pretrain_tmix_lnx_rkvres_xg_forward(x, r, k, v, residual_scale, weight, bias, g,
                                        head_size=64):
    """Reference lnx_rkvres_xg/pretrain_bf16_forward.cpp:75-98: returns (output, mean, rstd)."""
    return ops.pretrain_tmix_lnx_rkvres_xg_forward(x, r, k, v, residual_scale, weight, bias, g,
                                                   int(head_size))


def pretrain_tmix_lnx_rkvres_xg_backward(grad_output, x, r, k, v, residual_scale, weight, bias,
                                         g, mean, rstd, head_size=64):
    """Reference lnx_rkvres_xg/pretrain_bf16_backward.cpp:83-110: returns (grad_x, grad_r,
    grad_k, grad_v, grad_residual_scale, grad_weight, grad_bias, grad_g)."""
    return ops.pretrain_tmix_lnx_rkvres_xg_backward(grad_output, x, r, k, v, residual_scale,
                                                    weight, bias, g, mean, rstd,
                                                    int(head_size))

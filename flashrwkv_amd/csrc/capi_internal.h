// Internal helpers shared by the C-ABI translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>

#include "../../include/flashrwkv_amd.h"

namespace frwkv {

// Records a printf-style message as the calling thread's last error and
// returns status.
int set_error(int status, const char* fmt, ...);

// Converts a pending launch error into FRWKV_ERR_HIP with a message.
int check_launch(const char* what);

}  // namespace frwkv

// The replay stage on the per-token kernel (recurrent.hip), used by
// frwkv_chunk_replay for head sizes other than 64. Arguments as there.
int frwkv_replay_recurrent(int io_dtype, int decay_mode, int32_t num_chunks, int32_t num_heads,
                           int32_t head_size, int32_t total_tokens,
                           const int32_t* chunk_token_starts, const int32_t* chunk_token_ends,
                           const float* boundary, const void* r, const void* decay,
                           const void* decay_bias, const void* k, const void* v,
                           const void* a, const void* b, void* output, float* state_dot_a,
                           float scale, void* stream);

// Per-token training kernels (train_recurrent.hip) for head sizes 128 and
// 256, called by frwkv_statetune_{forward,backward,interior} and
// frwkv_pretrain_{forward,backward}. Chunks come either from segment arrays
// (seg_offsets/seg_starts/seg_ends of num_chunks chunks, dense_t = 0), from
// seg_starts/seg_ends alone with one chunk per unit (seg_offsets null; the
// fill pass), or, with dense_t > 0, from a dense [B, dense_t] layout in
// 16-token chunks with the pretraining checkpoint layout [B,H,T/16,D,D].
// state (forward) is S0 in / S_T out, or null for a zero start and no final
// state. interior holds the state at each 16-token piece start inside a
// chunk, at slot (piece start) / 16: written by the forward, read by the
// backward, which walks longer chunks piece by piece (without it a chunk
// longer than 16 tokens, or an out-of-range chunk, makes its unit's gradients
// NaN). slices: frwkv_train_slice_bytes of fp32 workspace (head size 256).
int frwkv_train_recurrent_forward(int io_dtype, int decay_mode, int32_t num_sequences,
                                  int32_t num_heads, int32_t head_size, int32_t total_tokens,
                                  const int32_t* seg_offsets, const int32_t* seg_starts,
                                  const int32_t* seg_ends, int32_t num_chunks, int32_t dense_t,
                                  float* state,
                                  const void* r, const void* decay, const void* decay_bias,
                                  const void* k, const void* v, const void* a, const void* b,
                                  void* output, float* boundary, float* state_dot_a,
                                  float* interior, int fill_only, float scale, void* stream);
int frwkv_train_recurrent_backward(int io_dtype, int decay_mode, int32_t num_sequences,
                                   int32_t num_heads, int32_t head_size, int32_t total_tokens,
                                   const int32_t* seg_offsets, const int32_t* seg_starts,
                                   const int32_t* seg_ends, int32_t num_chunks,
                                   int32_t dense_t, const float* boundary, const void* r, const void* decay,
                                   const void* decay_bias, const void* k, const void* v,
                                   const void* a, const void* b, const void* grad_output,
                                   const float* grad_final_state, void* grad_r,
                                   void* grad_decay, void* grad_k, void* grad_v, void* grad_a,
                                   void* grad_b, float* grad_initial_state,
                                   const float* interior, float* slices, float scale,
                                   void* stream);

// Bytes of the fp32 gradient slices the per-token backward needs at this head
// size (0 when a unit fits one workgroup, i.e. head size 128).
size_t frwkv_train_slice_bytes(int32_t head_size, int32_t num_heads, int32_t total_tokens);

// The recurrent operator's route for long sequences (chunk_fwd.hip): the
// split-precision chunk kernel on bf16 tokens, head size 64, fp32 pool.
// Arguments as frwkv_recurrent_forward's, already checked by it.
int frwkv_recurrent_chunked_forward(int decay_mode, int32_t num_sequences, int32_t num_heads,
                                    int32_t total_tokens, int32_t state_pool_size,
                                    const int32_t* cu_seqlens, const int32_t* state_indices,
                                    const int32_t* metadata_status, float* state_pool,
                                    const void* r, const void* decay, const void* decay_bias,
                                    const void* k, const void* v, const void* a, const void* b,
                                    void* output, float scale, void* stream);

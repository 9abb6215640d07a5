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

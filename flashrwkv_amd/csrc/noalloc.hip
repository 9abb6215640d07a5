// frwkv_statetune_backward_noalloc: frwkv_statetune_backward with its
// workspace in a file-scope device array instead of a caller buffer.
//
// The array lives in this translation unit, apart from the kernels, so that
// its code object holds nothing but the array: HIP loads a code object on a
// device when one of its symbols is first used there, and only this entry
// uses `scratch`. A process that never calls it does not pay for the array;
// one that does holds FRWKV_NOALLOC_SCRATCH_BYTES on each device it called
// it on, until the process ends. In host code the name `scratch` only stands
// for the symbol: its device address, per device, comes from
// hipGetSymbolAddress on the entry's first call with that device current,
// and only that address is handed to the kernels (as their workspace).

#include <mutex>

#include "capi_internal.h"

static __device__ __align__(256) unsigned char scratch[FRWKV_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_address[kMaxDevices] = {};

// Device address of this device's `scratch` (looked up once per device).
int scratch_address(void** out) {
  using namespace frwkv;
  int device = -1;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess || device < 0 || device >= kMaxDevices) {
    return set_error(FRWKV_ERR_HIP, "frwkv_statetune_backward_noalloc: no usable device (%s)",
                     hipGetErrorString(err));
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_address[device] == nullptr) {
    void* address = nullptr;
    err = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
    if (err != hipSuccess || address == nullptr) {
      return set_error(FRWKV_ERR_HIP,
                       "frwkv_statetune_backward_noalloc: scratch address on device %d: %s",
                       device, hipGetErrorString(err));
    }
    g_scratch_address[device] = address;
  }
  *out = g_scratch_address[device];
  return FRWKV_OK;
}

}  // namespace

extern "C" int frwkv_statetune_backward_noalloc(
    int io_dtype, int decay_mode, int32_t num_sequences, int32_t num_heads, int32_t head_size,
    int32_t total_tokens, int32_t num_chunks, const int32_t* sequence_chunk_offsets,
    const int32_t* chunk_token_starts, const int32_t* chunk_token_ends, const float* boundary,
    const float* interior, const void* r, const void* decay, const void* decay_bias,
    const void* k, const void* v, const void* a, const void* b, const void* grad_output,
    const float* grad_final_state, void* grad_r, void* grad_decay, void* grad_k, void* grad_v,
    void* grad_a, void* grad_b, float* grad_initial_state, float scale, void* stream) {
  using namespace frwkv;
  const size_t need = frwkv_statetune_backward_workspace_bytes(head_size, num_heads,
                                                               total_tokens, interior != nullptr);
  if (need > FRWKV_NOALLOC_SCRATCH_BYTES) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                     "frwkv_statetune_backward_noalloc: needs %zu bytes of scratch, the "
                     "static buffer holds %zu (pass the forward's interior states, or fewer "
                     "tokens or heads per call)",
                     need, static_cast<size_t>(FRWKV_NOALLOC_SCRATCH_BYTES));
  }
  void* work = nullptr;
  size_t work_bytes = 0;
  if (need > 0) {
    const int rc = scratch_address(&work);
    if (rc != FRWKV_OK) return rc;
    work_bytes = FRWKV_NOALLOC_SCRATCH_BYTES;
  }
  return frwkv_statetune_backward(io_dtype, decay_mode, num_sequences, num_heads, head_size,
                                  total_tokens, num_chunks, sequence_chunk_offsets,
                                  chunk_token_starts, chunk_token_ends, boundary, interior, r,
                                  decay, decay_bias, k, v, a, b, grad_output, grad_final_state,
                                  grad_r, grad_decay, grad_k, grad_v, grad_a, grad_b,
                                  grad_initial_state, work, work_bytes, scale, stream);
}

// Common C-ABI plumbing (status strings, per-thread error text) and the
// packed-metadata validation kernels.
//
// Metadata validation replaces the reference's validate_recurrent_metadata_kernel
// (csrc/validation/recurrent_metadata.cu:22-97): same status bits and the
// same snapshot semantics, but the duplicate-slot scan is spread over one
// workgroup per 256 sequences instead of one 256-thread block, so B up to
// 65535 stays cheap.
#include "capi_internal.h"

#include <cstdio>
#include <cstring>
#include <string>

namespace frwkv {

static thread_local std::string g_last_error;

int set_error(int status, const char* fmt, ...) {
  char buffer[512];
  va_list args;
  va_start(args, fmt);
  vsnprintf(buffer, sizeof(buffer), fmt, args);
  va_end(args);
  g_last_error = buffer;
  return status;
}

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return set_error(FRWKV_ERR_HIP, "%s: %s", what, hipGetErrorString(err));
  }
  return FRWKV_OK;
}

namespace {

constexpr int kMetaThreads = 256;

// Zeroes the status word and copies the caller's metadata into the snapshots.
__global__ __launch_bounds__(kMetaThreads) void metadata_snapshot_kernel(
    const int32_t* __restrict__ cu_seqlens, const int32_t* __restrict__ slots,
    int32_t num_sequences, int32_t* __restrict__ status,
    int32_t* __restrict__ cu_snapshot, int32_t* __restrict__ slot_snapshot) {
  const int stride = gridDim.x * blockDim.x;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i <= num_sequences;
       i += stride) {
    cu_snapshot[i] = cu_seqlens[i];
    if (i < num_sequences) slot_snapshot[i] = slots[i];
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) status[0] = 0;
}

// One thread per sequence: endpoint, range and slot-bound checks, plus the
// duplicate scan against every earlier sequence (tiles of earlier slots are
// staged through LDS). Errors are OR-ed in LDS, then once into status.
__global__ __launch_bounds__(kMetaThreads) void metadata_check_kernel(
    const int32_t* __restrict__ cu, const int32_t* __restrict__ slots,
    int32_t num_sequences, int32_t total_tokens, int32_t state_pool_size,
    int32_t* __restrict__ status) {
  __shared__ int32_t tile[kMetaThreads];
  __shared__ int32_t block_error;
  if (threadIdx.x == 0) block_error = 0;
  const int i = blockIdx.x * kMetaThreads + threadIdx.x;
  int error = 0;
  int32_t my_slot = -1;
  if (i < num_sequences) {
    if (i == 0 && (cu[0] != 0 || cu[num_sequences] != total_tokens)) {
      error |= FRWKV_META_BAD_ENDPOINT;
    }
    const int32_t start = cu[i];
    const int32_t end = cu[i + 1];
    if (start < 0 || end <= start || end > total_tokens) {
      error |= FRWKV_META_BAD_RANGE;
    }
    my_slot = slots[i];
    if (my_slot < 0 || my_slot >= state_pool_size) {
      error |= FRWKV_META_BAD_SLOT;
    }
  }
  __syncthreads();
  // Duplicate scan over tiles 0..blockIdx.x (earlier sequences only).
  const int last_tile = blockIdx.x;
  for (int t = 0; t <= last_tile; ++t) {
    const int j = t * kMetaThreads + threadIdx.x;
    tile[threadIdx.x] = j < num_sequences ? slots[j] : -1;
    __syncthreads();
    if (i < num_sequences && !(error & FRWKV_META_BAD_SLOT)) {
      const int limit = (t == last_tile) ? threadIdx.x : kMetaThreads;
      for (int q = 0; q < limit; ++q) {
        if (tile[q] == my_slot) {
          error |= FRWKV_META_DUPLICATE_SLOT;
          break;
        }
      }
    }
    __syncthreads();
  }
  if (error) atomicOr(&block_error, error);
  __syncthreads();
  if (threadIdx.x == 0 && block_error != 0) atomicOr(status, block_error);
}

}  // namespace
}  // namespace frwkv

extern "C" {

int frwkv_abi_version(void) { return FRWKV_ABI_VERSION; }

const char* frwkv_status_string(int status) {
  switch (status) {
    case FRWKV_OK:
      return "ok";
    case FRWKV_ERR_INVALID_ARGUMENT:
      return "invalid argument";
    case FRWKV_ERR_UNSUPPORTED:
      return "unsupported configuration";
    case FRWKV_ERR_HIP:
      return "HIP runtime error";
    default:
      return "unknown status";
  }
}

const char* frwkv_last_error(void) { return frwkv::g_last_error.c_str(); }

int frwkv_metadata_validate(const int32_t* cu_seqlens,
                            const int32_t* state_indices,
                            int32_t num_sequences, int32_t total_tokens,
                            int32_t state_pool_size, int32_t* status,
                            int32_t* cu_seqlens_snapshot,
                            int32_t* state_indices_snapshot, void* stream) {
  using namespace frwkv;
  if (!cu_seqlens || !state_indices || !status || !cu_seqlens_snapshot ||
      !state_indices_snapshot) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                     "frwkv_metadata_validate: null pointer argument");
  }
  if (num_sequences <= 0 || num_sequences > 65535) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                     "state_indices must contain 1..65535 sequences, got %d",
                     num_sequences);
  }
  if (total_tokens <= 0 || state_pool_size <= 0) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                     "total_tokens and state_pool_size must be positive");
  }
  auto s = static_cast<hipStream_t>(stream);
  const int blocks = (num_sequences + kMetaThreads) / kMetaThreads;
  hipLaunchKernelGGL(metadata_snapshot_kernel, dim3(blocks), dim3(kMetaThreads),
                     0, s, cu_seqlens, state_indices, num_sequences, status,
                     cu_seqlens_snapshot, state_indices_snapshot);
  int rc = check_launch("metadata_snapshot_kernel");
  if (rc != FRWKV_OK) return rc;
  const int check_blocks = (num_sequences + kMetaThreads - 1) / kMetaThreads;
  hipLaunchKernelGGL(metadata_check_kernel, dim3(check_blocks),
                     dim3(kMetaThreads), 0, s, cu_seqlens_snapshot,
                     state_indices_snapshot, num_sequences, total_tokens,
                     state_pool_size, status);
  return check_launch("metadata_check_kernel");
}

}  // extern "C"

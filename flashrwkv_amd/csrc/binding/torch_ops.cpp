// Thin PyTorch-ROCm binding over the flashrwkv_amd C ABI.
//
// Replaces the reference's pybind11 registration layer for the WKV7 path
// (csrc/registration.cpp:6-8, csrc/bindings.cpp:6-44 and the per-op register_*
// functions, e.g. csrc/sm120/tmix/wkv7/infer_recurrent_fp32io16_forward_varlen.cpp:314-362)
// with TORCH_LIBRARY(flashrwkv2) ops and a torch custom class for the
// metadata ticket. This layer only validates tensors (same rules and error
// vocabulary as csrc/validation.cpp:27-129 and the ticket checks of
// infer_recurrent_fp32io16_forward_varlen.cpp:44-202), owns allocations the
// reference binding owns (metadata snapshots, status word) and forwards raw
// device pointers plus the current HIP stream to libflashrwkv_amd.so.
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/custom_class.h>
#include <torch/library.h>

#include <hip/hip_runtime_api.h>

#include <atomic>
#include <cmath>
#include <cstdint>
#include <limits>
#include <optional>
#include <unordered_set>
#include <vector>

#include "../../../include/flashrwkv_amd.h"

namespace {

using at::Tensor;

void check_rc(int rc) {
  TORCH_CHECK(rc == FRWKV_OK, "flashrwkv_amd: ", frwkv_status_string(rc), ": ",
              frwkv_last_error());
}

void* current_stream(const Tensor& t) {
  return c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

// True while the current stream of t's device is being captured into a HIP
// graph. A query that fails (the legacy stream during another thread's
// global-mode capture) counts as capturing; its error is cleared so that the
// next launch check does not report it.
bool stream_is_capturing(const Tensor& t) {
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  const hipError_t err =
      hipStreamIsCapturing(static_cast<hipStream_t>(current_stream(t)), &status);
  if (err != hipSuccess) {
    (void)hipGetLastError();
    return true;
  }
  return status != hipStreamCaptureStatusNone;
}

// The chunked MFMA kernels (prefill, training forward and backward, replay)
// have not been run inside a captured HIP graph: the one capture of an
// autograd training step that held them ended in a host segmentation fault
// while the capture closed, cause not found. Ops that would launch them
// under capture therefore refuse with this error instead.
void refuse_capture(const Tensor& t, const char* op) {
  TORCH_CHECK(!stream_is_capturing(t), op,
              " does not run under HIP graph capture: its chunked kernels are not validated "
              "inside a captured graph; run it eagerly");
}

// Route of long bf16 sequences (head size 64, max_seqlen >= 64) in the
// fp32-state recurrent op: 0 the split-precision chunk kernel (default), 1
// the per-token fp32 kernel for every call, as the reference computes it.
std::atomic<int> g_recurrent_long_route{0};

void check_device_contiguous(const Tensor& t, const char* name) {
  TORCH_CHECK(t.is_cuda(), name, " must be CUDA");
  TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
}

void check_same_device(const Tensor& ref, const Tensor& t, const char* name) {
  TORCH_CHECK(t.device() == ref.device(), name,
              " must be on the same device as state");
}

int io_code(at::ScalarType dtype) {
  switch (dtype) {
    case at::kFloat:
      return FRWKV_DTYPE_F32;
    case at::kHalf:
      return FRWKV_DTYPE_F16;
    case at::kBFloat16:
      return FRWKV_DTYPE_BF16;
    default:
      TORCH_CHECK(false, "token tensors must be float16 or bfloat16");
  }
  return -1;
}

std::optional<uint32_t> tensor_version(const Tensor& t) {
  if (t.unsafeGetTensorImpl()->is_inference()) return std::nullopt;
  return t.unsafeGetTensorImpl()->version_counter().current_version();
}

// Host check of packed metadata values (one device-to-host copy). Returns the
// longest sequence. Same rules and messages as the reference's
// check_recurrent_metadata_values (infer_recurrent_fp32io16_forward_varlen.cpp:44-79).
int64_t check_metadata_values(const Tensor& cu_seqlens,
                              const Tensor& state_indices, int64_t total_tokens,
                              int64_t state_pool_size) {
  const Tensor cu = cu_seqlens.to(at::kCPU).contiguous();
  const Tensor slots = state_indices.to(at::kCPU).contiguous();
  const int32_t* offsets = cu.data_ptr<int32_t>();
  const int32_t* slot_ptr = slots.data_ptr<int32_t>();
  const int64_t count = slots.numel();
  TORCH_CHECK(offsets[0] == 0, "query_start_loc must start at 0");
  TORCH_CHECK(offsets[count] == total_tokens,
              "the final query_start_loc offset must equal total_tokens");
  std::unordered_set<int32_t> seen;
  int64_t longest = 0;
  for (int64_t i = 0; i < count; ++i) {
    const int32_t start = offsets[i];
    const int32_t end = offsets[i + 1];
    TORCH_CHECK(start >= 0 && end > start && end <= total_tokens,
                "query_start_loc must be strictly increasing with non-empty sequences");
    TORCH_CHECK(slot_ptr[i] >= 0 && slot_ptr[i] < state_pool_size,
                "state_indices entries must be within the state pool");
    TORCH_CHECK(seen.insert(slot_ptr[i]).second,
                "state_indices must be unique within one call");
    longest = std::max<int64_t>(longest, end - start);
  }
  return longest;
}

struct Prepared {
  Tensor cu_snapshot;
  Tensor slot_snapshot;
  Tensor status;
};

// Launches the device validation (status word + snapshots) on the current stream.
Prepared device_prepare(const Tensor& cu_seqlens, const Tensor& state_indices,
                        int64_t total_tokens, int64_t state_pool_size) {
  c10::DeviceGuard guard(cu_seqlens.device());
  Prepared p{at::empty_like(cu_seqlens), at::empty_like(state_indices),
             at::empty({1}, cu_seqlens.options())};
  check_rc(frwkv_metadata_validate(
      cu_seqlens.data_ptr<int32_t>(), state_indices.data_ptr<int32_t>(),
      static_cast<int32_t>(state_indices.numel()),
      static_cast<int32_t>(total_tokens), static_cast<int32_t>(state_pool_size),
      p.status.data_ptr<int32_t>(), p.cu_snapshot.data_ptr<int32_t>(),
      p.slot_snapshot.data_ptr<int32_t>(), current_stream(cu_seqlens)));
  return p;
}

// Reusable validated-metadata ticket (the reference's RecurrentMetadataTicket,
// infer_recurrent_fp32io16_forward_varlen.cpp:88-202): it pins the caller's
// metadata tensors by identity, data pointer, sizes, strides and version
// counter, the launch sizes, the device and the preparing stream, and holds
// the device snapshots and status word that launches read.
class MetadataTicket : public torch::CustomClassHolder {
 public:
  MetadataTicket(Tensor cu, Tensor slots, Prepared prepared, int64_t total_tokens,
                 int64_t state_pool_size, int64_t max_seqlen)
      : cu_(std::move(cu)),
        slots_(std::move(slots)),
        prepared_(std::move(prepared)),
        cu_version_(tensor_version(cu_)),
        slots_version_(tensor_version(slots_)),
        cu_data_(cu_.data_ptr()),
        slots_data_(slots_.data_ptr()),
        cu_sizes_(cu_.sizes().vec()),
        slots_sizes_(slots_.sizes().vec()),
        cu_strides_(cu_.strides().vec()),
        slots_strides_(slots_.strides().vec()),
        total_tokens_(total_tokens),
        state_pool_size_(state_pool_size),
        max_seqlen_(max_seqlen),
        device_(cu_.device()),
        stream_(current_stream(cu_)) {}

  void check_compatible(const Tensor& cu, const Tensor& slots,
                        int64_t total_tokens, int64_t state_pool_size,
                        int64_t max_seqlen) const {
    TORCH_CHECK(cu.is_same(cu_),
                "validated_metadata query_start_loc identity mismatch");
    TORCH_CHECK(slots.is_same(slots_),
                "validated_metadata state_indices identity mismatch");
    TORCH_CHECK(cu.data_ptr() == cu_data_ && slots.data_ptr() == slots_data_,
                "validated_metadata metadata data_ptr mismatch");
    TORCH_CHECK(cu.sizes().vec() == cu_sizes_ && slots.sizes().vec() == slots_sizes_ &&
                    cu.strides().vec() == cu_strides_ &&
                    slots.strides().vec() == slots_strides_,
                "validated_metadata metadata shape or stride mismatch");
    if (cu_version_.has_value()) {
      TORCH_CHECK(tensor_version(cu) == cu_version_,
                  "validated_metadata query_start_loc version mismatch");
    }
    if (slots_version_.has_value()) {
      TORCH_CHECK(tensor_version(slots) == slots_version_,
                  "validated_metadata state_indices version mismatch");
    }
    TORCH_CHECK(cu.device() == device_ && slots.device() == device_,
                "validated_metadata device mismatch");
    TORCH_CHECK(total_tokens == total_tokens_,
                "validated_metadata total_tokens mismatch");
    TORCH_CHECK(state_pool_size == state_pool_size_,
                "validated_metadata state_pool_size mismatch");
    if (max_seqlen > 0) {
      TORCH_CHECK(max_seqlen == max_seqlen_, "validated_metadata max_seqlen mismatch");
    }
    TORCH_CHECK(current_stream(cu) == stream_,
                "validated_metadata stream mismatch; prepare and consume the "
                "ticket on the same stream");
  }

  const Prepared& prepared() const { return prepared_; }
  int64_t max_seqlen() const { return max_seqlen_; }
  int64_t total_tokens() const { return total_tokens_; }
  int64_t state_pool_size() const { return state_pool_size_; }

 private:
  Tensor cu_, slots_;
  Prepared prepared_;
  std::optional<uint32_t> cu_version_, slots_version_;
  void* cu_data_;
  void* slots_data_;
  std::vector<int64_t> cu_sizes_, slots_sizes_, cu_strides_, slots_strides_;
  int64_t total_tokens_, state_pool_size_, max_seqlen_;
  c10::Device device_;
  void* stream_;
};

using TicketPtr = c10::intrusive_ptr<MetadataTicket>;

TicketPtr prepare_recurrent_metadata(Tensor query_start_loc, Tensor state_indices,
                                     int64_t total_tokens, int64_t state_pool_size,
                                     int64_t max_seqlen) {
  check_device_contiguous(query_start_loc, "query_start_loc");
  check_device_contiguous(state_indices, "state_indices");
  TORCH_CHECK(state_indices.device() == query_start_loc.device(),
              "state_indices must be on the same device as state");
  TORCH_CHECK(query_start_loc.scalar_type() == at::kInt &&
                  state_indices.scalar_type() == at::kInt,
              "recurrent metadata must be int32");
  TORCH_CHECK(query_start_loc.dim() == 1 && state_indices.dim() == 1 &&
                  state_indices.numel() > 0 &&
                  query_start_loc.numel() == state_indices.numel() + 1,
              "query_start_loc must have shape [B+1] and state_indices shape [B]");
  TORCH_CHECK(state_indices.numel() <= 65535,
              "state_indices must contain at most 65535 sequences");
  TORCH_CHECK(total_tokens > 0 && total_tokens <= std::numeric_limits<int32_t>::max(),
              "total_tokens must be positive and fit in int32");
  TORCH_CHECK(state_pool_size > 0 &&
                  state_pool_size <= std::numeric_limits<int32_t>::max(),
              "state_pool_size must be positive and fit in int32");
  const int64_t inferred =
      check_metadata_values(query_start_loc, state_indices, total_tokens, state_pool_size);
  if (max_seqlen <= 0) {
    max_seqlen = inferred;
  } else {
    TORCH_CHECK(max_seqlen == inferred,
                "max_seqlen must equal the largest packed sequence length");
  }
  Prepared prepared =
      device_prepare(query_start_loc, state_indices, total_tokens, state_pool_size);
  return c10::make_intrusive<MetadataTicket>(query_start_loc, state_indices,
                                             std::move(prepared), total_tokens,
                                             state_pool_size, max_seqlen);
}

// Layout checks of the fp32-state recurrent op (csrc/validation.cpp:27-129
// rules; fp32 tokens only through the internal op).
void check_recurrent_layout(const Tensor& cu, const Tensor& slots,
                            const Tensor& state, const Tensor& r,
                            const Tensor& decay, const Tensor& k, const Tensor& v,
                            const Tensor& a, const Tensor& b, const Tensor& output,
                            double scale, bool allow_fp32_tokens) {
  const std::pair<const Tensor*, const char*> all[] = {
      {&cu, "query_start_loc"}, {&slots, "state_indices"}, {&state, "state"},
      {&r, "r"}, {&decay, "decay_logits"}, {&k, "k"}, {&v, "v"}, {&a, "a"},
      {&b, "b"}, {&output, "output"}};
  for (const auto& item : all) check_device_contiguous(*item.first, item.second);
  TORCH_CHECK(cu.scalar_type() == at::kInt, "query_start_loc must be int32");
  TORCH_CHECK(slots.scalar_type() == at::kInt, "state_indices must be int32");
  TORCH_CHECK(std::isfinite(scale), "scale must be finite");
  const int64_t count = slots.numel();
  TORCH_CHECK(count > 0 && count <= 65535,
              "state_indices must contain 1..65535 sequences");
  TORCH_CHECK(slots.dim() == 1, "state_indices must have shape [N]");
  TORCH_CHECK(cu.dim() == 1 && cu.size(0) == count + 1,
              "query_start_loc must have shape [N+1]");
  TORCH_CHECK(state.dim() == 4 && state.size(0) > 0 && state.size(1) > 0 &&
                  state.size(2) == state.size(3),
              "state must have square shape [slots,H,D,D]");
  TORCH_CHECK(state.scalar_type() == at::kFloat, "state must be float32");
  const int64_t d = state.size(2);
  TORCH_CHECK(d == 64 || d == 128 || d == 256,
              "recurrent head size must be 64, 128, or 256, got ", d);
  TORCH_CHECK(state.size(0) <= std::numeric_limits<int32_t>::max(),
              "state slot count must fit in int32");
  const int64_t heads = state.size(1);
  TORCH_CHECK(r.dim() == 3 && r.size(0) > 0 && r.size(1) == heads && r.size(2) == d,
              "r must have shape [total_tokens,H,D] matching state");
  TORCH_CHECK(r.size(0) <= std::numeric_limits<int32_t>::max(),
              "token count must fit in int32");
  TORCH_CHECK(r.sizes() == decay.sizes() && r.sizes() == k.sizes() &&
                  r.sizes() == v.sizes() && r.sizes() == a.sizes() &&
                  r.sizes() == b.sizes() && r.sizes() == output.sizes(),
              "r,decay_logits,k,v,a,b,output shape mismatch");
  const bool ok_dtype = r.scalar_type() == at::kHalf ||
                        r.scalar_type() == at::kBFloat16 ||
                        (allow_fp32_tokens && r.scalar_type() == at::kFloat);
  TORCH_CHECK(ok_dtype, "token tensors must be float16 or bfloat16");
  const auto dt = r.scalar_type();
  TORCH_CHECK(decay.scalar_type() == dt && k.scalar_type() == dt &&
                  v.scalar_type() == dt && a.scalar_type() == dt &&
                  b.scalar_type() == dt && output.scalar_type() == dt,
              "r,decay_logits,k,v,a,b,output dtype mismatch");
  for (const auto& item : all) check_same_device(state, *item.first, item.second);
}

void check_decay_bias(const std::optional<Tensor>& bias, const Tensor& state,
                      const Tensor& r) {
  if (!bias.has_value()) return;
  check_device_contiguous(*bias, "decay_bias");
  check_same_device(state, *bias, "decay_bias");
  TORCH_CHECK(bias->scalar_type() == r.scalar_type(),
              "decay_bias must match the token tensor dtype");
  const int64_t heads = state.size(1), d = state.size(2);
  TORCH_CHECK((bias->dim() == 1 && bias->numel() == heads * d) ||
                  (bias->dim() == 2 && bias->size(0) == heads && bias->size(1) == d),
              "decay_bias must have shape [H*D] or [H,D]");
}

void recurrent_impl(const Tensor& cu, const Tensor& slots, Tensor& state,
                    const Tensor& r, const Tensor& decay, const Tensor& k,
                    const Tensor& v, const Tensor& a, const Tensor& b,
                    Tensor& output, double scale,
                    const std::optional<Tensor>& decay_bias,
                    const std::optional<TicketPtr>& ticket, int64_t max_seqlen,
                    int decay_mode, bool allow_fp32_tokens) {
  check_recurrent_layout(cu, slots, state, r, decay, k, v, a, b, output, scale,
                         allow_fp32_tokens);
  check_decay_bias(decay_bias, state, r);
  TORCH_CHECK(!(decay_bias.has_value() && decay_mode == FRWKV_DECAY_RAW_W),
              "decay_bias is only defined for decay logits");
  c10::DeviceGuard guard(state.device());
  Prepared launch;
  if (ticket.has_value() && ticket->defined()) {
    (*ticket)->check_compatible(cu, slots, r.size(0), state.size(0), max_seqlen);
    launch = (*ticket)->prepared();
    max_seqlen = (*ticket)->max_seqlen();
  } else {
    // No ticket: device validation only (no host sync); a direct call with
    // bad metadata fails closed inside the kernel.
    launch = device_prepare(cu, slots, r.size(0), state.size(0));
  }
  // A max_seqlen the library does not know sends every sequence to the
  // per-token fp32 kernel (the shape it uses for any max_seqlen above 2): when
  // the caller asked for that route, and under graph capture, where the chunk
  // kernels do not run.
  if (max_seqlen > 2 &&
      (g_recurrent_long_route.load(std::memory_order_relaxed) == 1 || stream_is_capturing(state))) {
    max_seqlen = -1;
  }
  check_rc(frwkv_recurrent_forward(
      io_code(r.scalar_type()), decay_mode, static_cast<int32_t>(slots.numel()),
      static_cast<int32_t>(state.size(1)), static_cast<int32_t>(state.size(2)),
      static_cast<int32_t>(r.size(0)), static_cast<int32_t>(max_seqlen),
      static_cast<int32_t>(state.size(0)), launch.cu_snapshot.data_ptr<int32_t>(),
      launch.slot_snapshot.data_ptr<int32_t>(), launch.status.data_ptr<int32_t>(),
      state.data_ptr<float>(), r.data_ptr(), decay.data_ptr(),
      decay_bias.has_value() ? decay_bias->data_ptr() : nullptr, k.data_ptr(),
      v.data_ptr(), a.data_ptr(), b.data_ptr(), output.data_ptr(),
      static_cast<float>(scale), current_stream(state)));
}

// Process-wide route of long bf16 sequences in the fp32-state op (not a
// reference op): 0 split-precision chunk kernel, 1 per-token fp32 kernel.
// Returns the previous route.
int64_t set_recurrent_long_route(int64_t route) {
  TORCH_CHECK(route == 0 || route == 1,
              "route must be 0 (split-precision chunk kernel) or 1 (per-token fp32 kernel)");
  return g_recurrent_long_route.exchange(static_cast<int>(route));
}

int64_t recurrent_long_route() { return g_recurrent_long_route.load(); }

// Public op: raw decay logits, fp16/bf16 tokens.
void recurrent_fp32_from_decay_logits(
    Tensor query_start_loc, Tensor state_indices, Tensor state, Tensor r,
    Tensor decay_logits, Tensor k, Tensor v, Tensor a, Tensor b, Tensor output,
    double scale, std::optional<Tensor> decay_bias,
    std::optional<TicketPtr> validated_metadata, int64_t max_seqlen) {
  recurrent_impl(query_start_loc, state_indices, state, r, decay_logits, k, v, a,
                 b, output, scale, decay_bias, validated_metadata, max_seqlen,
                 FRWKV_DECAY_LOGITS, /*allow_fp32_tokens=*/false);
}

// Internal op: explicit decay mode (0 logits, 1 raw retention) and fp32 tokens
// allowed. Used by the measurement harness and parity tests.
void recurrent_fp32_forward_internal(
    Tensor query_start_loc, Tensor state_indices, Tensor state, Tensor r,
    Tensor decay, Tensor k, Tensor v, Tensor a, Tensor b, Tensor output,
    double scale, int64_t decay_mode, std::optional<Tensor> decay_bias,
    std::optional<TicketPtr> validated_metadata, int64_t max_seqlen) {
  TORCH_CHECK(decay_mode == FRWKV_DECAY_LOGITS || decay_mode == FRWKV_DECAY_RAW_W,
              "decay_mode must be 0 (logits) or 1 (raw retention)");
  recurrent_impl(query_start_loc, state_indices, state, r, decay, k, v, a, b,
                 output, scale, decay_bias, validated_metadata, max_seqlen,
                 static_cast<int>(decay_mode), /*allow_fp32_tokens=*/true);
}

// ---------------------------------------------------------------- chunk ---

void check_chunk_tokens(const Tensor& r, const Tensor& decay, const Tensor& k,
                        const Tensor& v, const Tensor& a, const Tensor& b,
                        bool bf16_only, bool any_head_size = false) {
  const std::pair<const Tensor*, const char*> all[] = {
      {&r, "r"}, {&decay, "decay_logits"}, {&k, "k"}, {&v, "v"}, {&a, "a"}, {&b, "b"}};
  for (const auto& item : all) {
    check_device_contiguous(*item.first, item.second);
    TORCH_CHECK(item.first->device() == r.device(), item.second,
                " must be on the same device as r");
    if (bf16_only) {
      TORCH_CHECK(item.first->scalar_type() == at::kBFloat16, item.second,
                  " must be bfloat16");
    } else {
      TORCH_CHECK(item.first->scalar_type() == r.scalar_type(),
                  "r,decay_logits,k,v,a,b dtype mismatch");
    }
    TORCH_CHECK(item.first->sizes() == r.sizes(), item.second,
                " must have the same shape as r");
  }
  TORCH_CHECK(r.scalar_type() == at::kBFloat16 || r.scalar_type() == at::kHalf,
              "token tensors must be float16 or bfloat16");
  if (any_head_size) {
    TORCH_CHECK(r.dim() == 3 && r.size(0) > 0 && r.size(1) > 0 &&
                    (r.size(2) == 64 || r.size(2) == 128 || r.size(2) == 256),
                "token tensors must have shape [total_tokens,H,D], D in {64,128,256}");
  } else {
    TORCH_CHECK(r.dim() == 3 && r.size(0) > 0 && r.size(1) > 0 && r.size(2) == 64,
                "chunk token tensors must have shape [total_tokens,H,64]");
  }
  TORCH_CHECK(r.size(0) <= std::numeric_limits<int32_t>::max(),
              "token count must fit in int32");
}

void check_chunk_metadata(const Tensor& cu, const Tensor& slots, const Tensor& r) {
  check_device_contiguous(cu, "cu_seqlens");
  check_device_contiguous(slots, "state_indices");
  TORCH_CHECK(cu.device() == r.device() && slots.device() == r.device(),
              "cu_seqlens and state_indices must be on the same device as r");
  TORCH_CHECK(cu.scalar_type() == at::kInt && slots.scalar_type() == at::kInt,
              "chunk metadata must be int32");
  TORCH_CHECK(cu.dim() == 1 && slots.dim() == 1 && slots.numel() > 0 &&
                  cu.numel() == slots.numel() + 1,
              "cu_seqlens must have shape [B+1] and state_indices [B]");
  TORCH_CHECK(slots.numel() <= 65535, "state_indices must contain at most 65535 sequences");
}

void chunk_impl(const Tensor& r, const Tensor& decay, const Tensor& k, const Tensor& v,
                const Tensor& a, const Tensor& b, Tensor& pool, const Tensor& cu,
                const Tensor& slots, double scale, const std::optional<Tensor>& decay_bias,
                int decay_mode, const Tensor& output) {
  TORCH_CHECK(std::isfinite(scale), "scale must be finite");
  check_device_contiguous(pool, "state_pool");
  TORCH_CHECK(pool.device() == r.device(), "state_pool must be on the same device as r");
  TORCH_CHECK(pool.dim() == 4 && pool.size(0) > 0 && pool.size(1) == r.size(1) &&
                  pool.size(2) == 64 && pool.size(3) == 64,
              "state_pool must have shape [slots,H,64,64]");
  TORCH_CHECK(pool.size(0) <= std::numeric_limits<int32_t>::max(),
              "state slot count must fit in int32");
  check_chunk_metadata(cu, slots, r);
  check_decay_bias(decay_bias, pool, r);
  TORCH_CHECK(!(decay_bias.has_value() && decay_mode == FRWKV_DECAY_RAW_W),
              "decay_bias is only defined for decay logits");
  const int pool_code = pool.scalar_type() == at::kFloat      ? FRWKV_DTYPE_F32
                        : pool.scalar_type() == at::kBFloat16 ? FRWKV_DTYPE_BF16
                                                              : -1;
  TORCH_CHECK(pool_code >= 0, "state_pool must be float32 or bfloat16");
  c10::DeviceGuard guard(r.device());
  refuse_capture(r, "the chunked WKV7 forward");
  Prepared launch = device_prepare(cu, slots, r.size(0), pool.size(0));
  check_rc(frwkv_chunk_forward(
      io_code(r.scalar_type()), decay_mode, pool_code, static_cast<int32_t>(slots.numel()),
      static_cast<int32_t>(r.size(1)), 64, static_cast<int32_t>(r.size(0)),
      static_cast<int32_t>(pool.size(0)), launch.cu_snapshot.data_ptr<int32_t>(),
      launch.slot_snapshot.data_ptr<int32_t>(), launch.status.data_ptr<int32_t>(),
      pool.data_ptr(), r.data_ptr(), decay.data_ptr(),
      decay_bias.has_value() ? decay_bias->data_ptr() : nullptr, k.data_ptr(), v.data_ptr(),
      a.data_ptr(), b.data_ptr(), output.data_ptr(), static_cast<float>(scale),
      current_stream(r)));
}

// Public op (reference infer_chunk_bf16_forward_varlen.cpp:77-171): bf16
// tokens, bf16 pool updated in place, returns (output, state_pool).
std::tuple<Tensor, Tensor> infer_chunk_bf16_forward_varlen(
    Tensor r, Tensor decay_logits, Tensor k, Tensor v, Tensor a, Tensor b,
    Tensor state_pool, Tensor cu_seqlens, Tensor state_indices, int64_t chunk_size,
    int64_t max_seqlen, double scale, std::optional<Tensor> decay_bias) {
  check_chunk_tokens(r, decay_logits, k, v, a, b, /*bf16_only=*/true);
  TORCH_CHECK(state_pool.scalar_type() == at::kBFloat16, "state_pool must be bfloat16");
  TORCH_CHECK(chunk_size > 0, "chunk_size must be positive");
  TORCH_CHECK(max_seqlen > 0, "max_seqlen must be positive");
  Tensor output = at::empty_like(v);
  chunk_impl(r, decay_logits, k, v, a, b, state_pool, cu_seqlens, state_indices, scale,
             decay_bias, FRWKV_DECAY_LOGITS, output);
  return {output, state_pool};
}

// Internal op: explicit decay mode, fp16/bf16 tokens, fp32 or bf16 pool.
Tensor chunk_forward_internal(Tensor r, Tensor decay, Tensor k, Tensor v, Tensor a,
                              Tensor b, Tensor state_pool, Tensor cu_seqlens,
                              Tensor state_indices, double scale, int64_t decay_mode,
                              std::optional<Tensor> decay_bias) {
  TORCH_CHECK(decay_mode == FRWKV_DECAY_LOGITS || decay_mode == FRWKV_DECAY_RAW_W,
              "decay_mode must be 0 (logits) or 1 (raw retention)");
  check_chunk_tokens(r, decay, k, v, a, b, /*bf16_only=*/false);
  Tensor output = at::empty_like(v);
  chunk_impl(r, decay, k, v, a, b, state_pool, cu_seqlens, state_indices, scale, decay_bias,
             static_cast<int>(decay_mode), output);
  return output;
}

// ------------------------------------------------------------ statetune ---

// The interior-state buffer of the training ops, or none: a float32 tensor of
// at least frwkv_statetune_interior_bytes bytes, opaque storage
// ([ceil(N/P), H, D, D] fp32 with P = 64 at head size 64, else 16; bf16 states
// at head size 128).
float* checked_interior(const std::optional<Tensor>& interior, const Tensor& r, int64_t d) {
  if (!interior.has_value() || !interior->defined()) return nullptr;
  check_device_contiguous(*interior, "interior");
  TORCH_CHECK(interior->device() == r.device(), "interior must share the token device");
  const size_t need = frwkv_statetune_interior_bytes(
      static_cast<int32_t>(d), static_cast<int32_t>(r.size(1)), static_cast<int32_t>(r.size(0)));
  TORCH_CHECK(interior->scalar_type() == at::kFloat &&
                  static_cast<size_t>(interior->numel()) * sizeof(float) >= need,
              "interior must be float32 with at least ", need, " bytes");
  return interior->data_ptr<float>();
}

// Device scratch of the given size from PyTorch's caching allocator (on the
// current stream), or an undefined tensor for 0 bytes.
Tensor workspace_like(const Tensor& like, size_t bytes) {
  if (bytes == 0) return Tensor();
  return at::empty({static_cast<int64_t>(bytes)}, like.options().dtype(at::kByte));
}

void check_statetune_metadata(const Tensor& offsets, const Tensor& starts,
                              const Tensor& ends, const Tensor& state) {
  const std::pair<const Tensor*, const char*> all[] = {
      {&offsets, "sequence_chunk_offsets"},
      {&starts, "chunk_token_starts"},
      {&ends, "chunk_token_ends"}};
  for (const auto& item : all) {
    check_device_contiguous(*item.first, item.second);
    TORCH_CHECK(item.first->scalar_type() == at::kInt, item.second, " must be int32");
    TORCH_CHECK(item.first->device() == state.device(), item.second,
                " must share the state device");
    TORCH_CHECK(item.first->dim() == 1, item.second, " must be one-dimensional");
  }
  TORCH_CHECK(offsets.numel() == state.size(0) + 1,
              "sequence_chunk_offsets must have shape [B+1]");
  TORCH_CHECK(starts.numel() > 0 && ends.numel() == starts.numel(),
              "chunk token metadata must have matching shape [C]");
}

void statetune_forward_impl(const Tensor& offsets, const Tensor& starts, const Tensor& ends,
                            Tensor& state, const Tensor& r, const Tensor& decay,
                            const Tensor& k, const Tensor& v, const Tensor& a,
                            const Tensor& b, Tensor& output, Tensor& boundary,
                            Tensor& state_dot_a, const std::optional<Tensor>& interior,
                            double scale, int decay_mode) {
  TORCH_CHECK(std::isfinite(scale), "scale must be finite");
  check_device_contiguous(state, "state");
  TORCH_CHECK(state.scalar_type() == at::kFloat, "state must be float32");
  TORCH_CHECK(state.dim() == 4 && state.size(0) > 0 && state.size(1) > 0 &&
                  state.size(2) == state.size(3),
              "state must have shape [B,H,D,D]");
  const int64_t d = state.size(2);
  TORCH_CHECK(d == 64 || d == 128 || d == 256, "state head size must be 64, 128, or 256");
  check_chunk_tokens(r, decay, k, v, a, b, /*bf16_only=*/false, /*any_head_size=*/true);
  TORCH_CHECK(r.size(1) == state.size(1) && r.size(2) == d,
              "token tensors must have shape [total_tokens,H,D]");
  for (const auto* t : {&r, &decay, &k, &v, &a, &b}) check_same_device(state, *t, "token");
  check_statetune_metadata(offsets, starts, ends, state);
  check_device_contiguous(output, "output");
  check_device_contiguous(boundary, "boundary");
  check_device_contiguous(state_dot_a, "state_dot_a");
  TORCH_CHECK(output.sizes() == r.sizes() && output.scalar_type() == r.scalar_type(),
              "output must match r");
  TORCH_CHECK(boundary.scalar_type() == at::kFloat && boundary.dim() == 4 &&
                  boundary.size(0) == starts.numel() && boundary.size(1) == state.size(1) &&
                  boundary.size(2) == d && boundary.size(3) == d,
              "boundary must have shape [chunks,H,D,D] float32");
  TORCH_CHECK(state_dot_a.scalar_type() == at::kFloat && state_dot_a.sizes() == r.sizes(),
              "state_dot_a must have shape [total_tokens,H,D] float32");
  float* interior_ptr = checked_interior(interior, r, d);
  c10::DeviceGuard guard(state.device());
  refuse_capture(r, "the StateTune forward");
  check_rc(frwkv_statetune_forward(
      io_code(r.scalar_type()), decay_mode, static_cast<int32_t>(state.size(0)),
      static_cast<int32_t>(state.size(1)), static_cast<int32_t>(d), static_cast<int32_t>(r.size(0)),
      static_cast<int32_t>(starts.numel()), offsets.data_ptr<int32_t>(),
      starts.data_ptr<int32_t>(), ends.data_ptr<int32_t>(), state.data_ptr<float>(),
      r.data_ptr(), decay.data_ptr(), nullptr, k.data_ptr(), v.data_ptr(), a.data_ptr(),
      b.data_ptr(), output.data_ptr(), boundary.data_ptr<float>(),
      state_dot_a.data_ptr<float>(), interior_ptr, static_cast<float>(scale),
      current_stream(state)));
}

// Reference statetune_recurrent_fp32io16_forward.cpp:26-44 (decay logits).
void statetune_recurrent_fp32io16_forward(Tensor offsets, Tensor starts, Tensor ends,
                                          Tensor state, Tensor r, Tensor decay_logits,
                                          Tensor k, Tensor v, Tensor a, Tensor b,
                                          Tensor output, Tensor boundary,
                                          Tensor state_dot_a, double scale) {
  statetune_forward_impl(offsets, starts, ends, state, r, decay_logits, k, v, a, b, output,
                         boundary, state_dot_a, std::nullopt, scale, FRWKV_DECAY_LOGITS);
}

void statetune_forward_internal(Tensor offsets, Tensor starts, Tensor ends, Tensor state,
                                Tensor r, Tensor decay, Tensor k, Tensor v, Tensor a,
                                Tensor b, Tensor output, Tensor boundary,
                                Tensor state_dot_a, std::optional<Tensor> interior, double scale,
                                int64_t decay_mode) {
  TORCH_CHECK(decay_mode == FRWKV_DECAY_LOGITS || decay_mode == FRWKV_DECAY_RAW_W,
              "decay_mode must be 0 (logits) or 1 (raw retention)");
  statetune_forward_impl(offsets, starts, ends, state, r, decay, k, v, a, b, output,
                         boundary, state_dot_a, interior, scale, static_cast<int>(decay_mode));
}

// Reference statetune_recurrent_fp32io16_backward.cpp:34-82: optional
// gradient outputs (allocated here when omitted), final_state and
// state_dot_a accepted for contract compatibility (the recompute-based
// backward does not need them).
void statetune_backward_impl(const Tensor& offsets, const Tensor& starts, const Tensor& ends,
                             const Tensor& r, const Tensor& decay, const Tensor& k,
                             const Tensor& v, const Tensor& a, const Tensor& b,
                             const std::optional<Tensor>& grad_output,
                             const std::optional<Tensor>& grad_final_state,
                             const Tensor& boundary, std::optional<Tensor> grad_r,
                             std::optional<Tensor> grad_decay, std::optional<Tensor> grad_k,
                             std::optional<Tensor> grad_v, std::optional<Tensor> grad_a,
                             std::optional<Tensor> grad_b,
                             std::optional<Tensor> grad_initial_state, int64_t num_sequences,
                             const std::optional<Tensor>& interior, double scale,
                             int decay_mode) {
  TORCH_CHECK(std::isfinite(scale), "scale must be finite");
  check_chunk_tokens(r, decay, k, v, a, b, /*bf16_only=*/false, /*any_head_size=*/true);
  const int64_t heads = r.size(1), d = r.size(2);
  TORCH_CHECK(d == 64 || d == 128 || d == 256, "token head size must be 64, 128, or 256");
  check_device_contiguous(boundary, "boundary");
  TORCH_CHECK(boundary.scalar_type() == at::kFloat && boundary.dim() == 4 &&
                  boundary.size(0) == starts.numel() && boundary.size(1) == heads &&
                  boundary.size(2) == d && boundary.size(3) == d,
              "boundary must have shape [chunks,H,D,D] float32");
  for (const auto* t : {&offsets, &starts, &ends}) {
    check_device_contiguous(*t, "chunk metadata");
    TORCH_CHECK(t->scalar_type() == at::kInt && t->dim() == 1, "chunk metadata must be int32 1-D");
    TORCH_CHECK(t->device() == r.device(), "chunk metadata must share the token device");
  }
  TORCH_CHECK(offsets.numel() == num_sequences + 1,
              "sequence_chunk_offsets must have shape [B+1]");
  TORCH_CHECK(starts.numel() > 0 && ends.numel() == starts.numel(),
              "chunk token metadata must have matching shape [C]");
  if (grad_output.has_value() && grad_output->defined()) {
    check_device_contiguous(*grad_output, "grad_output");
    TORCH_CHECK(grad_output->sizes() == r.sizes() && grad_output->scalar_type() == r.scalar_type(),
                "grad_output must match r");
  }
  const auto state_opts = r.options().dtype(at::kFloat);
  if (grad_final_state.has_value() && grad_final_state->defined()) {
    check_device_contiguous(*grad_final_state, "grad_final_state");
    TORCH_CHECK(grad_final_state->scalar_type() == at::kFloat &&
                    grad_final_state->dim() == 4 && grad_final_state->size(0) == num_sequences &&
                    grad_final_state->size(1) == heads && grad_final_state->size(2) == d &&
                    grad_final_state->size(3) == d,
                "grad_final_state must have shape [B,H,D,D] float32");
  }
  auto token_grad = [&](std::optional<Tensor>& t, const char* name) {
    if (!t.has_value() || !t->defined()) t = at::empty_like(r);
    check_device_contiguous(*t, name);
    TORCH_CHECK(t->sizes() == r.sizes() && t->scalar_type() == r.scalar_type(), name,
                " must match r");
    return t->data_ptr();
  };
  void* gr = token_grad(grad_r, "grad_r");
  void* gd = token_grad(grad_decay, "grad_decay_logits");
  void* gk = token_grad(grad_k, "grad_k");
  void* gv = token_grad(grad_v, "grad_v");
  void* ga = token_grad(grad_a, "grad_a");
  void* gb = token_grad(grad_b, "grad_b");
  if (!grad_initial_state.has_value() || !grad_initial_state->defined()) {
    grad_initial_state = at::empty({num_sequences, heads, d, d}, state_opts);
  }
  check_device_contiguous(*grad_initial_state, "grad_initial_state");
  TORCH_CHECK(grad_initial_state->scalar_type() == at::kFloat &&
                  grad_initial_state->numel() == num_sequences * heads * d * d,
              "grad_initial_state must have shape [B,H,D,D] float32");
  const float* interior_ptr = checked_interior(interior, r, d);
  c10::DeviceGuard guard(r.device());
  refuse_capture(r, "the StateTune backward");
  const bool has_dy = grad_output.has_value() && grad_output->defined();
  const bool has_ds = grad_final_state.has_value() && grad_final_state->defined();
  // Without the forward's interior states the call recomputes them into the
  // workspace (chunks longer than one piece only), so any chunk length works.
  const size_t ws_bytes = frwkv_statetune_backward_workspace_bytes(
      static_cast<int32_t>(d), static_cast<int32_t>(heads), static_cast<int32_t>(r.size(0)),
      interior_ptr != nullptr);
  Tensor ws = workspace_like(r, ws_bytes);
  check_rc(frwkv_statetune_backward(
      io_code(r.scalar_type()), decay_mode, static_cast<int32_t>(num_sequences),
      static_cast<int32_t>(heads), static_cast<int32_t>(d), static_cast<int32_t>(r.size(0)),
      static_cast<int32_t>(starts.numel()), offsets.data_ptr<int32_t>(),
      starts.data_ptr<int32_t>(), ends.data_ptr<int32_t>(), boundary.data_ptr<float>(),
      interior_ptr, r.data_ptr(), decay.data_ptr(), nullptr, k.data_ptr(), v.data_ptr(),
      a.data_ptr(), b.data_ptr(), has_dy ? grad_output->data_ptr() : nullptr,
      has_ds ? grad_final_state->data_ptr<float>() : nullptr, gr, gd, gk, gv, ga, gb,
      grad_initial_state->data_ptr<float>(), ws.defined() ? ws.data_ptr() : nullptr, ws_bytes,
      static_cast<float>(scale), current_stream(r)));
}

void statetune_recurrent_fp32io16_backward(
    Tensor offsets, Tensor starts, Tensor ends, Tensor final_state, Tensor r,
    Tensor decay_logits, Tensor k, Tensor v, Tensor a, Tensor b, Tensor state_dot_a,
    std::optional<Tensor> grad_output, std::optional<Tensor> grad_final_state, Tensor boundary,
    std::optional<Tensor> grad_r, std::optional<Tensor> grad_decay_logits,
    std::optional<Tensor> grad_k, std::optional<Tensor> grad_v, std::optional<Tensor> grad_a,
    std::optional<Tensor> grad_b, std::optional<Tensor> grad_initial_state, double scale) {
  (void)state_dot_a;
  check_device_contiguous(final_state, "final_state");
  statetune_backward_impl(offsets, starts, ends, r, decay_logits, k, v, a, b, grad_output,
                          grad_final_state, boundary, grad_r, grad_decay_logits, grad_k,
                          grad_v, grad_a, grad_b, grad_initial_state, final_state.size(0),
                          std::nullopt, scale, FRWKV_DECAY_LOGITS);
}

void statetune_backward_internal(
    Tensor offsets, Tensor starts, Tensor ends, Tensor r, Tensor decay, Tensor k, Tensor v,
    Tensor a, Tensor b, std::optional<Tensor> grad_output,
    std::optional<Tensor> grad_final_state, Tensor boundary, Tensor grad_r, Tensor grad_decay,
    Tensor grad_k, Tensor grad_v, Tensor grad_a, Tensor grad_b, Tensor grad_initial_state,
    std::optional<Tensor> interior, double scale, int64_t decay_mode) {
  TORCH_CHECK(decay_mode == FRWKV_DECAY_LOGITS || decay_mode == FRWKV_DECAY_RAW_W,
              "decay_mode must be 0 (logits) or 1 (raw retention)");
  statetune_backward_impl(offsets, starts, ends, r, decay, k, v, a, b, grad_output,
                          grad_final_state, boundary, grad_r, grad_decay, grad_k, grad_v,
                          grad_a, grad_b, grad_initial_state, offsets.numel() - 1, interior,
                          scale, static_cast<int>(decay_mode));
}

// ---------------------------------------------------------------------------
// rwkv7_clampw_v3 (pretraining): reference
// csrc/sm90/tmix/wkv7/pretrain_recurrent_bf16_forward.cpp:20-53. Dense
// [B,T,H,D] tokens with clampw decay logits, S0 = 0, no final state; s is the
// state every 16 tokens [B,H,T/16,D,D] fp32 and sa is a^T S_{t-1} [B,T,H,D]
// fp32. Head size 64 runs the chunked MFMA kernels, 128 and 256 the
// per-token training kernels.

void check_clampw_tokens(const std::vector<std::pair<const Tensor*, const char*>>& all,
                         int64_t head_size) {
  TORCH_CHECK(head_size == 64 || head_size == 128 || head_size == 256,
              "head_size must be one of 64, 128, or 256");
  const Tensor& r = *all[0].first;
  TORCH_CHECK(r.dim() == 4 && r.size(3) == head_size,
              "input head dimension must equal head_size");
  for (const auto& item : all) {
    check_device_contiguous(*item.first, item.second);
    TORCH_CHECK(item.first->device() == r.device(), item.second,
                " must be on the same device as r");
    TORCH_CHECK(item.first->scalar_type() == r.scalar_type(),
                "r,w,k,v,a,b dtype mismatch");
    TORCH_CHECK(item.first->sizes() == r.sizes(), item.second,
                " must have the same shape as r");
  }
  TORCH_CHECK(r.scalar_type() == at::kBFloat16 || r.scalar_type() == at::kHalf,
              "token tensors must be float16 or bfloat16");
  TORCH_CHECK(r.size(0) > 0 && r.size(1) > 0 && r.size(2) > 0 && r.size(1) % 16 == 0,
              "tokens must have shape [B,T,H,D] with T a positive multiple of 16");
  TORCH_CHECK(r.size(0) * r.size(1) <= std::numeric_limits<int32_t>::max(),
              "B * T must fit int32");
}

void check_clampw_side(const Tensor& r, const Tensor& s, const Tensor& sa) {
  const int64_t B = r.size(0), T = r.size(1), H = r.size(2), D = r.size(3);
  check_device_contiguous(s, "s");
  check_device_contiguous(sa, "sa");
  TORCH_CHECK(s.device() == r.device() && sa.device() == r.device(),
              "s and sa must be on the same device as r");
  TORCH_CHECK(s.scalar_type() == at::kFloat && s.dim() == 5 && s.size(0) == B &&
                  s.size(1) == H && s.size(2) == T / 16 && s.size(3) == D && s.size(4) == D,
              "s must have shape [B,H,T/16,D,D] float32");
  TORCH_CHECK(sa.scalar_type() == at::kFloat && sa.sizes() == r.sizes(),
              "sa must have shape [B,T,H,D] float32");
}

void clampw_forward(Tensor r, Tensor w, Tensor k, Tensor v, Tensor a, Tensor b, Tensor y,
                    Tensor s, Tensor sa, int64_t head_size) {
  check_clampw_tokens({{&r, "r"}, {&w, "w"}, {&k, "k"}, {&v, "v"}, {&a, "a"}, {&b, "b"},
                       {&y, "y"}}, head_size);
  check_clampw_side(r, s, sa);
  c10::DeviceGuard guard(r.device());
  refuse_capture(r, "the clampw-v3 pretraining forward");
  check_rc(frwkv_pretrain_forward(
      io_code(r.scalar_type()), FRWKV_DECAY_LOGITS, static_cast<int32_t>(r.size(0)),
      static_cast<int32_t>(r.size(1)), static_cast<int32_t>(r.size(2)),
      static_cast<int32_t>(head_size), r.data_ptr(), w.data_ptr(), k.data_ptr(), v.data_ptr(),
      a.data_ptr(), b.data_ptr(), y.data_ptr(), s.data_ptr<float>(), sa.data_ptr<float>(),
      current_stream(r)));
}

void clampw_backward(Tensor r, Tensor w, Tensor k, Tensor v, Tensor a, Tensor b, Tensor dy,
                     Tensor s, Tensor sa, Tensor dr, Tensor dw, Tensor dk, Tensor dv, Tensor da,
                     Tensor db, int64_t head_size) {
  check_clampw_tokens({{&r, "r"}, {&w, "w"}, {&k, "k"}, {&v, "v"}, {&a, "a"}, {&b, "b"},
                       {&dy, "dy"}, {&dr, "dr"}, {&dw, "dw"}, {&dk, "dk"}, {&dv, "dv"},
                       {&da, "da"}, {&db, "db"}}, head_size);
  check_clampw_side(r, s, sa);
  c10::DeviceGuard guard(r.device());
  const size_t ws_bytes = frwkv_pretrain_backward_workspace_bytes(
      static_cast<int32_t>(r.size(0)), static_cast<int32_t>(r.size(1)),
      static_cast<int32_t>(r.size(2)), static_cast<int32_t>(head_size));
  refuse_capture(r, "the clampw-v3 pretraining backward");
  Tensor ws = workspace_like(r, ws_bytes);
  check_rc(frwkv_pretrain_backward(
      io_code(r.scalar_type()), FRWKV_DECAY_LOGITS, static_cast<int32_t>(r.size(0)),
      static_cast<int32_t>(r.size(1)), static_cast<int32_t>(r.size(2)),
      static_cast<int32_t>(head_size), r.data_ptr(), w.data_ptr(), k.data_ptr(), v.data_ptr(),
      a.data_ptr(), b.data_ptr(), dy.data_ptr(), s.data_ptr<float>(), dr.data_ptr(),
      dw.data_ptr(), dk.data_ptr(), dv.data_ptr(), da.data_ptr(), db.data_ptr(),
      ws.defined() ? ws.data_ptr() : nullptr, ws_bytes, current_stream(r)));
}

// ---------------------------------------------------------------------------
// RL/infctx chunk family: reference
// csrc/sm90/rl_infctx/wkv7/rl_infctx_chunk_fp32io16_forward.cpp:70-233 and
// rl_infctx_chunk_fp32io16_backward.cpp:20-128. The forward's result does not
// depend on the caller's chunking or strategy (both are validated): head size
// 64 runs the chunked kernel, 128 and 256 the fp32 per-token kernel, on a
// working copy of the state.

// Host check of the chunk metadata (one small device-to-host copy, as in the
// reference); returns the per-sequence token offsets [B+1].
std::vector<int32_t> check_rl_chunk_metadata(const Tensor& offsets, const Tensor& starts,
                                             const Tensor& ends, int64_t num_sequences,
                                             int64_t total_tokens, const Tensor& state) {
  const std::pair<const Tensor*, const char*> all[] = {
      {&offsets, "sequence_chunk_offsets"},
      {&starts, "chunk_token_starts"},
      {&ends, "chunk_token_ends"}};
  for (const auto& item : all) {
    check_device_contiguous(*item.first, item.second);
    TORCH_CHECK(item.first->device() == state.device(), item.second,
                " must be on the same device as state");
    TORCH_CHECK(item.first->scalar_type() == at::kInt, item.second, " must be int32");
  }
  TORCH_CHECK(offsets.dim() == 1 && offsets.numel() == num_sequences + 1,
              "sequence_chunk_offsets must have shape [B+1]");
  TORCH_CHECK(starts.dim() == 1 && starts.numel() > 0 && starts.sizes() == ends.sizes(),
              "chunk token metadata must have matching shape [C]");
  TORCH_CHECK(starts.numel() * state.size(1) <= std::numeric_limits<int>::max(),
              "chunk/head grid must fit in int32");
  const Tensor seq_cpu = offsets.to(at::kCPU).contiguous();
  const Tensor starts_cpu = starts.to(at::kCPU).contiguous();
  const Tensor ends_cpu = ends.to(at::kCPU).contiguous();
  const int32_t* seq = seq_cpu.data_ptr<int32_t>();
  const int32_t* st = starts_cpu.data_ptr<int32_t>();
  const int32_t* en = ends_cpu.data_ptr<int32_t>();
  const int64_t chunks = starts.numel();
  TORCH_CHECK(seq[0] == 0 && seq[num_sequences] == chunks,
              "sequence_chunk_offsets must cover all chunks");
  std::vector<int32_t> cu(num_sequences + 1, 0);
  int32_t previous_end = 0;
  for (int64_t s = 0; s < num_sequences; ++s) {
    const int32_t c0 = seq[s], c1 = seq[s + 1];
    TORCH_CHECK(c0 >= 0 && c1 > c0 && c1 <= chunks,
                "each sequence must own at least one ordered chunk");
    TORCH_CHECK(st[c0] == previous_end, "chunks must cover packed tokens without gaps");
    for (int32_t c = c0; c < c1; ++c) {
      TORCH_CHECK(st[c] >= 0 && en[c] > st[c] && en[c] <= total_tokens &&
                      (c == c0 || st[c] == en[c - 1]),
                  "chunk token ranges must be contiguous and non-empty");
    }
    cu[s] = st[c0];
    previous_end = en[c1 - 1];
  }
  TORCH_CHECK(previous_end == total_tokens, "chunks must cover exactly all packed tokens");
  cu[num_sequences] = previous_end;
  return cu;
}

std::tuple<Tensor, Tensor> rl_infctx_forward(Tensor offsets, Tensor starts, Tensor ends,
                                             Tensor state, Tensor r, Tensor decay_logits,
                                             Tensor k, Tensor v, Tensor a, Tensor b,
                                             int64_t strategy, double scale,
                                             std::optional<Tensor> decay_bias) {
  TORCH_CHECK(strategy == 0 || strategy == 1,
              "strategy must be 0 (materialized) or 1 (recompute)");
  TORCH_CHECK(state.is_cuda() && state.is_contiguous() && state.scalar_type() == at::kFloat,
              "RL/Infctx state must be contiguous CUDA float32");
  TORCH_CHECK(state.dim() == 4 && state.size(0) > 0 && state.size(1) > 0 &&
                  state.size(2) == state.size(3) &&
                  (state.size(2) == 64 || state.size(2) == 128 || state.size(2) == 256),
              "RL/Infctx state must have shape [B,H,D,D], D in {64,128,256}");
  const int64_t batch = state.size(0);
  TORCH_CHECK(r.dim() == 3, "RL/Infctx token tensors must have shape [N,H,D]");
  const std::vector<int32_t> cu_host =
      check_rl_chunk_metadata(offsets, starts, ends, batch, r.size(0), state);
  c10::DeviceGuard guard(state.device());
  Tensor working = state.clone();
  Tensor output = at::empty_like(v);
  const Tensor cu = at::tensor(cu_host, at::TensorOptions().dtype(at::kInt)).to(state.device());
  const Tensor slots = at::arange(batch, at::TensorOptions().dtype(at::kInt).device(state.device()));
  if (state.size(2) == 64) {
    check_chunk_tokens(r, decay_logits, k, v, a, b, /*bf16_only=*/false);
    chunk_impl(r, decay_logits, k, v, a, b, working, cu, slots, scale, decay_bias,
               FRWKV_DECAY_LOGITS, output);
  } else {
    int64_t max_len = 0;
    for (int64_t s = 0; s < batch; ++s) max_len = std::max<int64_t>(max_len, cu_host[s + 1] - cu_host[s]);
    recurrent_impl(cu, slots, working, r, decay_logits, k, v, a, b, output, scale, decay_bias,
                   std::nullopt, max_len, FRWKV_DECAY_LOGITS, /*allow_fp32_tokens=*/false);
  }
  return {output, working};
}

void rl_infctx_replay(Tensor starts, Tensor ends, Tensor boundary, Tensor r, Tensor decay_logits,
                      Tensor k, Tensor v, Tensor a, Tensor b, Tensor output, Tensor state_dot_a,
                      double scale, std::optional<Tensor> decay_bias) {
  for (const auto* t : {&boundary, &r, &decay_logits, &k, &v, &a, &b, &output, &state_dot_a,
                        &starts, &ends}) {
    check_device_contiguous(*t, "replay tensors");
  }
  TORCH_CHECK(std::isfinite(scale), "scale must be finite");
  TORCH_CHECK(starts.scalar_type() == at::kInt && ends.scalar_type() == at::kInt,
              "chunk token metadata must be int32");
  TORCH_CHECK(starts.dim() == 1 && starts.numel() > 0 && starts.sizes() == ends.sizes(),
              "chunk token metadata must have shape [C]");
  TORCH_CHECK(r.dim() == 3 && r.size(0) > 0 &&
                  (r.size(2) == 64 || r.size(2) == 128 || r.size(2) == 256),
              "replay token tensors must have shape [N,H,D], D in {64,128,256}");
  TORCH_CHECK(boundary.dim() == 4 && boundary.size(0) == starts.numel() &&
                  boundary.size(1) == r.size(1) && boundary.size(2) == r.size(2) &&
                  boundary.size(3) == r.size(2) && boundary.scalar_type() == at::kFloat,
              "boundary must have shape [C,H,D,D] and be float32");
  const std::pair<const Tensor*, const char*> toks[] = {
      {&decay_logits, "decay_logits"}, {&k, "k"}, {&v, "v"}, {&a, "a"}, {&b, "b"},
      {&output, "output"}};
  for (const auto& item : toks) {
    TORCH_CHECK(item.first->sizes() == r.sizes(), item.second, " must match r shape");
    TORCH_CHECK(item.first->scalar_type() == r.scalar_type(), item.second, " must match r dtype");
    TORCH_CHECK(item.first->device() == r.device(), item.second,
                " must be on the same device as r");
  }
  TORCH_CHECK(r.scalar_type() == at::kHalf || r.scalar_type() == at::kBFloat16,
              "replay token tensors must be float16 or bfloat16");
  TORCH_CHECK(state_dot_a.sizes() == r.sizes() && state_dot_a.scalar_type() == at::kFloat,
              "state_dot_a must match r shape and be float32");
  for (const auto* t : {&starts, &ends, &boundary, &state_dot_a}) {
    TORCH_CHECK(t->device() == r.device(), "replay metadata/workspace must be on the same device as r");
  }
  if (decay_bias.has_value()) {
    check_device_contiguous(*decay_bias, "decay_bias");
    TORCH_CHECK(decay_bias->device() == r.device(), "decay_bias must be on the same device as r");
    TORCH_CHECK(decay_bias->scalar_type() == r.scalar_type(), "decay_bias must match r dtype");
    TORCH_CHECK((decay_bias->dim() == 1 && decay_bias->numel() == r.size(1) * r.size(2)) ||
                    (decay_bias->dim() == 2 && decay_bias->size(0) == r.size(1) &&
                     decay_bias->size(1) == r.size(2)),
                "decay_bias must have shape [H*D] or [H,D]");
  }
  c10::DeviceGuard guard(r.device());
  refuse_capture(r, "the RL/Infctx replay");
  check_rc(frwkv_chunk_replay(
      io_code(r.scalar_type()), FRWKV_DECAY_LOGITS, static_cast<int32_t>(starts.numel()),
      static_cast<int32_t>(r.size(1)), static_cast<int32_t>(r.size(2)),
      static_cast<int32_t>(r.size(0)), starts.data_ptr<int32_t>(), ends.data_ptr<int32_t>(),
      boundary.data_ptr<float>(), r.data_ptr(), decay_logits.data_ptr(),
      decay_bias.has_value() ? decay_bias->data_ptr() : nullptr, k.data_ptr(), v.data_ptr(),
      a.data_ptr(), b.data_ptr(), output.data_ptr(), state_dot_a.data_ptr<float>(),
      static_cast<float>(scale), current_stream(r)));
}

// ------------------------------------------------------- fp16 state ---

// Layout checks of the fp16-state op: the rules and messages of the reference's
// check_fp16_recurrent_layout (infer_recurrent_fp16_forward_varlen.cpp:50-125).
void check_fp16_layout(const Tensor& cu, const Tensor& slots, const Tensor& elapsed,
                       const Tensor& state, const Tensor& r, const Tensor& decay,
                       const Tensor& k, const Tensor& v, const Tensor& a, const Tensor& b,
                       const Tensor& output, double scale) {
  const std::pair<const Tensor*, const char*> all[] = {
      {&cu, "query_start_loc"}, {&slots, "state_indices"},
      {&elapsed, "elapsed_state_pool"}, {&state, "state"}, {&r, "r"},
      {&decay, "decay_logits"}, {&k, "k"}, {&v, "v"}, {&a, "a"}, {&b, "b"},
      {&output, "output"}};
  for (const auto& item : all) check_device_contiguous(*item.first, item.second);
  for (const auto& item : all) check_same_device(state, *item.first, item.second);
  TORCH_CHECK(cu.scalar_type() == at::kInt && slots.scalar_type() == at::kInt &&
                  elapsed.scalar_type() == at::kInt,
              "recurrent metadata must be int32");
  TORCH_CHECK(slots.dim() == 1 && slots.numel() > 0 && cu.dim() == 1 &&
                  cu.numel() == slots.numel() + 1,
              "query_start_loc must have shape [B+1] and state_indices shape [B]");
  TORCH_CHECK(slots.numel() <= 65535, "state_indices must contain at most 65535 sequences");
  TORCH_CHECK(elapsed.dim() == 1 && state.dim() >= 1 && elapsed.size(0) == state.size(0),
              "elapsed_state_pool must have shape [state_pool_slots]");
  TORCH_CHECK(state.dim() == 4 && state.scalar_type() == at::kHalf && state.size(0) > 0 &&
                  state.size(1) > 0 && state.size(2) == state.size(3),
              "state must be contiguous float16 [slots,H,D,D]");
  TORCH_CHECK(state.size(0) <= std::numeric_limits<int32_t>::max(),
              "state slot count must fit in int32");
  const int64_t d = state.size(2);
  TORCH_CHECK(d == 64 || d == 128 || d == 256,
              "recurrent head size must be 64, 128, or 256, got ", d);
  TORCH_CHECK(r.dim() == 3 && r.size(0) > 0 && r.size(1) == state.size(1) && r.size(2) == d,
              "r must have packed shape [total_tokens,H,D] matching state");
  TORCH_CHECK(r.size(0) <= std::numeric_limits<int32_t>::max(),
              "token count must fit in int32");
  TORCH_CHECK(r.sizes() == decay.sizes() && r.sizes() == k.sizes() &&
                  r.sizes() == v.sizes() && r.sizes() == a.sizes() &&
                  r.sizes() == b.sizes() && r.sizes() == output.sizes(),
              "r,decay_logits,k,v,a,b,output shape mismatch");
  TORCH_CHECK(r.scalar_type() == at::kHalf && decay.scalar_type() == at::kHalf &&
                  k.scalar_type() == at::kHalf && v.scalar_type() == at::kHalf &&
                  a.scalar_type() == at::kHalf && b.scalar_type() == at::kHalf &&
                  output.scalar_type() == at::kHalf,
              "FP16-state recurrent token tensors must be float16");
  TORCH_CHECK(std::isfinite(scale), "scale must be finite");
}

// The reference's recurrent_fp16_from_decay_logits
// (infer_recurrent_fp16_forward_varlen.cpp:210-270).
void recurrent_fp16_from_decay_logits(
    Tensor query_start_loc, Tensor state_indices, Tensor elapsed_state_pool, Tensor state,
    Tensor r, Tensor decay_logits, Tensor k, Tensor v, Tensor a, Tensor b, Tensor output,
    double scale, std::optional<Tensor> decay_bias,
    std::optional<TicketPtr> validated_metadata, int64_t max_seqlen) {
  check_fp16_layout(query_start_loc, state_indices, elapsed_state_pool, state, r,
                    decay_logits, k, v, a, b, output, scale);
  if (decay_bias.has_value()) {
    check_device_contiguous(*decay_bias, "decay_bias");
    check_same_device(state, *decay_bias, "decay_bias");
    const int64_t heads = state.size(1), d = state.size(2);
    TORCH_CHECK(decay_bias->scalar_type() == at::kHalf &&
                    ((decay_bias->dim() == 1 && decay_bias->numel() == heads * d) ||
                     (decay_bias->dim() == 2 && decay_bias->size(0) == heads &&
                      decay_bias->size(1) == d)),
                "decay_bias must be float16 with shape [H*D] or [H,D]");
  }
  c10::DeviceGuard guard(state.device());
  Prepared launch;
  if (validated_metadata.has_value() && validated_metadata->defined()) {
    (*validated_metadata)
        ->check_compatible(query_start_loc, state_indices, r.size(0), state.size(0), max_seqlen);
    launch = (*validated_metadata)->prepared();
    max_seqlen = (*validated_metadata)->max_seqlen();
  } else {
    launch = device_prepare(query_start_loc, state_indices, r.size(0), state.size(0));
  }
  check_rc(frwkv_recurrent_fp16_forward(
      static_cast<int32_t>(state_indices.numel()), static_cast<int32_t>(state.size(1)),
      static_cast<int32_t>(state.size(2)), static_cast<int32_t>(r.size(0)),
      static_cast<int32_t>(max_seqlen), static_cast<int32_t>(state.size(0)),
      launch.cu_snapshot.data_ptr<int32_t>(), launch.slot_snapshot.data_ptr<int32_t>(),
      launch.status.data_ptr<int32_t>(), elapsed_state_pool.data_ptr<int32_t>(),
      state.data_ptr(), r.data_ptr(), decay_logits.data_ptr(),
      decay_bias.has_value() ? decay_bias->data_ptr() : nullptr, k.data_ptr(), v.data_ptr(),
      a.data_ptr(), b.data_ptr(), output.data_ptr(), static_cast<float>(scale),
      current_stream(state)));
}

// The reference's recurrent_fp16_advance_i32 (infer_recurrent_fp16_forward_varlen.cpp:129-135,
// range check .cu:1218-1219).
void recurrent_fp16_advance_i32(Tensor elapsed_state, int64_t amount) {
  check_device_contiguous(elapsed_state, "elapsed state");
  TORCH_CHECK(elapsed_state.scalar_type() == at::kInt,
              "elapsed state must be contiguous CUDA int32");
  TORCH_CHECK(elapsed_state.numel() > 0, "elapsed state must be non-empty");
  TORCH_CHECK(amount >= std::numeric_limits<int32_t>::min() &&
                  amount <= std::numeric_limits<int32_t>::max(),
              "advance_i32 amount out of int range");
  c10::DeviceGuard guard(elapsed_state.device());
  check_rc(frwkv_advance_i32(elapsed_state.data_ptr<int32_t>(), elapsed_state.numel(),
                             static_cast<int32_t>(amount), current_stream(elapsed_state)));
}

// The reference's recurrent_fp16_advance_i32_varlen
// (infer_recurrent_fp16_forward_varlen.cpp:137-191).
void recurrent_fp16_advance_i32_varlen(Tensor query_start_loc, Tensor state_indices,
                                       Tensor elapsed_state, int64_t total_tokens,
                                       std::optional<TicketPtr> validated_metadata) {
  check_device_contiguous(query_start_loc, "query_start_loc");
  check_device_contiguous(state_indices, "state_indices");
  check_device_contiguous(elapsed_state, "elapsed_state_pool");
  check_same_device(elapsed_state, query_start_loc, "query_start_loc");
  check_same_device(elapsed_state, state_indices, "state_indices");
  TORCH_CHECK(query_start_loc.scalar_type() == at::kInt &&
                  state_indices.scalar_type() == at::kInt &&
                  elapsed_state.scalar_type() == at::kInt,
              "varlen elapsed metadata must be contiguous CUDA int32");
  TORCH_CHECK(query_start_loc.dim() == 1 && state_indices.dim() == 1 &&
                  state_indices.numel() > 0 &&
                  query_start_loc.numel() == state_indices.numel() + 1,
              "query_start_loc must have shape [B+1] and state_indices shape [B]");
  TORCH_CHECK(state_indices.numel() <= 65535,
              "state_indices must contain at most 65535 sequences");
  TORCH_CHECK(elapsed_state.dim() == 1 && elapsed_state.size(0) > 0 && total_tokens > 0 &&
                  total_tokens <= std::numeric_limits<int32_t>::max() &&
                  elapsed_state.size(0) <= std::numeric_limits<int32_t>::max(),
              "invalid varlen elapsed state or total_tokens");
  c10::DeviceGuard guard(elapsed_state.device());
  Prepared launch;
  if (validated_metadata.has_value() && validated_metadata->defined()) {
    (*validated_metadata)
        ->check_compatible(query_start_loc, state_indices, total_tokens, elapsed_state.size(0),
                           -1);
    launch = (*validated_metadata)->prepared();
  } else {
    launch = device_prepare(query_start_loc, state_indices, total_tokens, elapsed_state.size(0));
  }
  check_rc(frwkv_advance_i32_varlen(
      static_cast<int32_t>(state_indices.numel()), static_cast<int32_t>(elapsed_state.size(0)),
      launch.cu_snapshot.data_ptr<int32_t>(), launch.slot_snapshot.data_ptr<int32_t>(),
      launch.status.data_ptr<int32_t>(), elapsed_state.data_ptr<int32_t>(),
      current_stream(elapsed_state)));
}

// The reference's recurrent_add_vec_forward_varlen (infer_recurrent_fp16_forward_varlen.cpp:193-208).
Tensor recurrent_add_vec_forward_varlen(Tensor x, Tensor vec) {
  check_device_contiguous(x, "x");
  check_device_contiguous(vec, "vec");
  TORCH_CHECK(vec.device() == x.device(), "vec must be on the same device as x");
  TORCH_CHECK(x.scalar_type() == at::kHalf && vec.scalar_type() == at::kHalf,
              "x and vec must be float16");
  TORCH_CHECK(x.dim() == 2 && x.size(0) > 0 && x.size(1) > 0 && x.size(1) % 2 == 0 &&
                  x.size(1) <= std::numeric_limits<int32_t>::max(),
              "x must have packed shape [total_tokens,C] with even C");
  TORCH_CHECK(vec.dim() == 1 && vec.size(0) == x.size(1), "vec must have shape [C]");
  c10::DeviceGuard guard(x.device());
  Tensor out = at::empty_like(x);
  check_rc(frwkv_add_vec(x.size(0), static_cast<int32_t>(x.size(1)), x.data_ptr(),
                         vec.data_ptr(), out.data_ptr(), current_stream(x)));
  return out;
}

}  // namespace

// ------------------------------------------- TMix producer and consumer ---

void check_half(const Tensor& t, const Tensor& ref, const char* name) {
  check_device_contiguous(t, name);
  TORCH_CHECK(t.device() == ref.device(), name, " must be on the same device as ",
              &ref == &t ? "itself" : "the first input");
  TORCH_CHECK(t.scalar_type() == at::kHalf, name, " must be float16");
}

void check_gate_common(const Tensor& x, const char* name, int64_t head_size,
                       int64_t batch_size, int64_t max_seqlen) {
  TORCH_CHECK(head_size == 64 || head_size == 128 || head_size == 256,
              "head_size must be one of 64, 128, or 256");
  TORCH_CHECK(x.dim() == 2 && x.size(0) > 0 && x.size(1) > 0 && x.size(1) % head_size == 0,
              name, " must have packed shape [total_tokens,H*head_size]");
  TORCH_CHECK(batch_size > 0, "batch_size must be positive");
  TORCH_CHECK(max_seqlen > 0, "max_seqlen must be positive");
}

// ------------------------------------------- lnx_rkvres_xg (training) ---
// Reference pretrain_tmix_lnx_rkvres_xg_forward / _backward
// (csrc/sm90/tmix/lnx_rkvres_xg/pretrain_bf16_forward.cpp:24-88,
// pretrain_bf16_backward.cpp:24-99): the same checks, in the same order, with
// the same messages.

void check_lnx_bf16(const Tensor& t, const char* name) {
  TORCH_CHECK(t.is_cuda() && t.is_contiguous() && t.scalar_type() == at::kBFloat16, name,
              " must be contiguous CUDA bfloat16");
}

void check_lnx_train_inputs(const Tensor& x, const Tensor& r, const Tensor& k,
                            const Tensor& v, const Tensor& residual_scale,
                            const Tensor& weight, const Tensor& bias, const Tensor& g,
                            int64_t head_size) {
  TORCH_CHECK(head_size == 64 || head_size == 128 || head_size == 256,
              "head_size must be one of 64, 128, or 256");
  const std::pair<const Tensor*, const char*> all[] = {
      {&x, "x"}, {&r, "r"}, {&k, "k"}, {&v, "v"}, {&residual_scale, "residual_scale"},
      {&weight, "weight"}, {&bias, "bias"}, {&g, "g"}};
  for (const auto& item : all) check_lnx_bf16(*item.first, item.second);
  TORCH_CHECK(x.dim() == 3 && x.size(0) > 0 && x.size(1) > 0 && x.size(2) > 0 &&
                  x.size(2) % head_size == 0,
              "x must have shape [B,T,C] with C divisible by head_size");
  for (const auto* t : {&r, &k, &v, &g}) {
    TORCH_CHECK(t->sizes() == x.sizes(), "token tensors must match x");
  }
  const int64_t heads = x.size(2) / head_size;
  TORCH_CHECK(residual_scale.dim() == 2 && residual_scale.size(0) == heads &&
                  residual_scale.size(1) == head_size,
              "residual_scale must have shape [C/head_size,head_size]");
  TORCH_CHECK(weight.dim() == 1 && bias.dim() == 1 && weight.size(0) == x.size(2) &&
                  bias.size(0) == x.size(2),
              "weight and bias must have shape [C]");
  for (const auto* t : {&r, &k, &v, &residual_scale, &weight, &bias, &g}) {
    TORCH_CHECK(t->device() == x.device(), "lnx tensors must share a device");
  }
}

std::tuple<Tensor, Tensor, Tensor> pretrain_tmix_lnx_rkvres_xg_forward(
    Tensor x, Tensor r, Tensor k, Tensor v, Tensor residual_scale, Tensor weight, Tensor bias,
    Tensor g, int64_t head_size) {
  check_lnx_train_inputs(x, r, k, v, residual_scale, weight, bias, g, head_size);
  c10::DeviceGuard guard(x.device());
  const int64_t heads = x.size(2) / head_size;
  Tensor out = at::empty_like(x);
  Tensor mean = at::empty({x.size(0), x.size(1), heads}, x.options().dtype(at::kFloat));
  Tensor rstd = at::empty_like(mean);
  check_rc(frwkv_lnx_pretrain_forward(
      FRWKV_DTYPE_BF16, x.size(0) * x.size(1), static_cast<int32_t>(heads),
      static_cast<int32_t>(head_size), x.data_ptr(), r.data_ptr(), k.data_ptr(), v.data_ptr(),
      residual_scale.data_ptr(), weight.data_ptr(), bias.data_ptr(), g.data_ptr(),
      out.data_ptr(), mean.data_ptr<float>(), rstd.data_ptr<float>(), current_stream(x)));
  return {out, mean, rstd};
}

std::vector<Tensor> pretrain_tmix_lnx_rkvres_xg_backward(
    Tensor grad_output, Tensor x, Tensor r, Tensor k, Tensor v, Tensor residual_scale,
    Tensor weight, Tensor bias, Tensor g, Tensor mean, Tensor rstd, int64_t head_size) {
  TORCH_CHECK(head_size == 64 || head_size == 128 || head_size == 256,
              "head_size must be one of 64, 128, or 256");
  const std::pair<const Tensor*, const char*> all[] = {
      {&grad_output, "grad_output"}, {&x, "x"}, {&r, "r"}, {&k, "k"}, {&v, "v"},
      {&residual_scale, "residual_scale"}, {&weight, "weight"}, {&bias, "bias"}, {&g, "g"}};
  for (const auto& item : all) check_lnx_bf16(*item.first, item.second);
  TORCH_CHECK(x.dim() == 3 && x.size(2) > 0 && x.size(2) % head_size == 0,
              "x must have shape [B,T,C] with C divisible by head_size");
  for (const auto* t : {&grad_output, &r, &k, &v, &g}) {
    TORCH_CHECK(t->sizes() == x.sizes(), "lnx token tensors must match x");
  }
  const int64_t heads = x.size(2) / head_size;
  TORCH_CHECK(residual_scale.dim() == 2 && residual_scale.size(0) == heads &&
                  residual_scale.size(1) == head_size,
              "residual_scale must have shape [C/head_size,head_size]");
  TORCH_CHECK(weight.dim() == 1 && weight.size(0) == x.size(2) && bias.sizes() == weight.sizes(),
              "weight and bias must have shape [C]");
  TORCH_CHECK(mean.dim() == 3 && mean.size(0) == x.size(0) && mean.size(1) == x.size(1) &&
                  mean.size(2) == heads && rstd.sizes() == mean.sizes() &&
                  mean.scalar_type() == at::kFloat && rstd.scalar_type() == at::kFloat,
              "mean and rstd must be float32 [B,T,C/head_size]");
  TORCH_CHECK(x.device() == mean.device() && x.device() == rstd.device(),
              "lnx tensors must share a device");
  for (const auto* t : {&grad_output, &r, &k, &v, &residual_scale, &weight, &bias, &g}) {
    TORCH_CHECK(t->device() == x.device(), "lnx tensors must share a device");
  }
  check_device_contiguous(mean, "mean");
  check_device_contiguous(rstd, "rstd");
  c10::DeviceGuard guard(x.device());
  Tensor gx = at::empty_like(x), gr = at::empty_like(x), gk = at::empty_like(x),
         gv = at::empty_like(x), gg = at::empty_like(x);
  Tensor g_rk = at::empty_like(residual_scale), g_w = at::empty_like(weight),
         g_b = at::empty_like(weight);
  const int64_t tokens = x.size(0) * x.size(1);
  const size_t ws_bytes = frwkv_lnx_pretrain_backward_workspace_bytes(
      tokens, static_cast<int32_t>(heads), static_cast<int32_t>(head_size));
  Tensor ws = workspace_like(x, ws_bytes);
  check_rc(frwkv_lnx_pretrain_backward(
      FRWKV_DTYPE_BF16, tokens, static_cast<int32_t>(heads), static_cast<int32_t>(head_size),
      grad_output.data_ptr(), x.data_ptr(), r.data_ptr(), k.data_ptr(), v.data_ptr(),
      residual_scale.data_ptr(), weight.data_ptr(), bias.data_ptr(), g.data_ptr(),
      mean.data_ptr<float>(), rstd.data_ptr<float>(), gx.data_ptr(), gr.data_ptr(),
      gk.data_ptr(), gv.data_ptr(), g_rk.data_ptr(), g_w.data_ptr(), g_b.data_ptr(),
      gg.data_ptr(), ws.defined() ? ws.data_ptr() : nullptr, ws_bytes, current_stream(x)));
  return {gx, gr, gk, gv, g_rk, g_w, g_b, gg};
}

// Reference tmix_kk_a_gate_forward_varlen (kk_a_gate/infer_fp16_forward_varlen.cpp:41-75).
std::tuple<Tensor, Tensor, Tensor> tmix_kk_a_gate_forward_varlen(
    Tensor k, Tensor k_k, Tensor a0, Tensor a12, Tensor k_a, int64_t head_size,
    int64_t batch_size, int64_t max_seqlen) {
  check_half(k, k, "k");
  check_gate_common(k, "k", head_size, batch_size, max_seqlen);
  const int64_t channels = k.size(1);
  const std::pair<const Tensor*, const char*> vectors[] = {
      {&k_k, "k_k"}, {&a0, "a0"}, {&k_a, "k_a"}};
  for (const auto& item : vectors) {
    check_half(*item.first, k, item.second);
    TORCH_CHECK(item.first->dim() == 1 && item.first->size(0) == channels, item.second,
                " must have shape [C]");
  }
  check_half(a12, k, "a12");
  TORCH_CHECK(a12.sizes() == k.sizes(), "a12 must match k's packed shape");
  c10::DeviceGuard guard(k.device());
  Tensor new_k = at::empty_like(k), neg_kk = at::empty_like(k), kka = at::empty_like(k);
  check_rc(frwkv_kk_a_gate(FRWKV_DTYPE_F16, k.size(0),
                           static_cast<int32_t>(channels / head_size),
                           static_cast<int32_t>(head_size), k.data_ptr(), k_k.data_ptr(),
                           a0.data_ptr(), a12.data_ptr(), k_a.data_ptr(), new_k.data_ptr(),
                           neg_kk.data_ptr(), kka.data_ptr(), current_stream(k)));
  return {new_k, neg_kk, kka};
}

// Reference tmix_lnx_rkvres_xg_forward_varlen (lnx_rkvres_xg/infer_fp16_forward_varlen.cpp:40-89).
Tensor tmix_lnx_rkvres_xg_forward_varlen(Tensor x, Tensor r, Tensor k, Tensor v, Tensor r_k,
                                         Tensor weight, Tensor bias, Tensor g,
                                         int64_t head_size, int64_t batch_size,
                                         int64_t max_seqlen) {
  check_half(x, x, "x");
  check_gate_common(x, "x", head_size, batch_size, max_seqlen);
  const int64_t channels = x.size(1);
  const std::pair<const Tensor*, const char*> tokens[] = {
      {&r, "r"}, {&k, "k"}, {&v, "v"}, {&g, "g"}};
  for (const auto& item : tokens) {
    check_half(*item.first, x, item.second);
    TORCH_CHECK(item.first->sizes() == x.sizes(), item.second, " must match x's packed shape");
  }
  const std::pair<const Tensor*, const char*> vectors[] = {
      {&r_k, "r_k"}, {&weight, "weight"}, {&bias, "bias"}};
  for (const auto& item : vectors) {
    check_half(*item.first, x, item.second);
    TORCH_CHECK(item.first->dim() == 1 && item.first->size(0) == channels, item.second,
                " must have shape [C]");
  }
  c10::DeviceGuard guard(x.device());
  Tensor out = at::empty_like(x);
  check_rc(frwkv_lnx_rkvres_xg(FRWKV_DTYPE_F16, x.size(0),
                               static_cast<int32_t>(channels / head_size),
                               static_cast<int32_t>(head_size), x.data_ptr(), r.data_ptr(),
                               k.data_ptr(), v.data_ptr(), r_k.data_ptr(), weight.data_ptr(),
                               bias.data_ptr(), g.data_ptr(), out.data_ptr(),
                               current_stream(x)));
  return out;
}

// Fused chain (no reference counterpart): kk_a_gate -> WKV7 step -> lnx_rkvres_xg.
// Token tensors [N,H,64] fp16/bf16, vectors [H*64] of the same dtype, fp32
// pool [slots,H,64,64] updated in place; returns the consumer's output.
Tensor recurrent_tmix_fused_forward(Tensor query_start_loc, Tensor state_indices,
                                    Tensor state, Tensor r, Tensor decay, Tensor k, Tensor v,
                                    Tensor a12, Tensor g, Tensor k_k, Tensor a0, Tensor k_a,
                                    Tensor r_k, Tensor ln_weight, Tensor ln_bias, double scale,
                                    int64_t decay_mode, std::optional<Tensor> decay_bias,
                                    std::optional<TicketPtr> validated_metadata) {
  TORCH_CHECK(decay_mode == FRWKV_DECAY_LOGITS || decay_mode == FRWKV_DECAY_RAW_W,
              "decay_mode must be 0 (logits) or 1 (raw retention)");
  Tensor output = at::empty_like(v);
  // The layout checks of the recurrent op, with a12 and g in the a and b places.
  check_recurrent_layout(query_start_loc, state_indices, state, r, decay, k, v, a12, g, output,
                         scale, /*allow_fp32_tokens=*/false);
  TORCH_CHECK(state.size(2) == 64, "the fused TMix chain supports head size 64, got ",
              state.size(2));
  const int64_t channels = state.size(1) * 64;
  const std::pair<const Tensor*, const char*> vectors[] = {
      {&k_k, "k_k"}, {&a0, "a0"}, {&k_a, "k_a"},
      {&r_k, "r_k"}, {&ln_weight, "ln_weight"}, {&ln_bias, "ln_bias"}};
  for (const auto& item : vectors) {
    check_device_contiguous(*item.first, item.second);
    check_same_device(state, *item.first, item.second);
    TORCH_CHECK(item.first->scalar_type() == r.scalar_type(), item.second,
                " must match the token tensor dtype");
    TORCH_CHECK(item.first->numel() == channels, item.second, " must have shape [H*D]");
  }
  check_decay_bias(decay_bias, state, r);
  TORCH_CHECK(!(decay_bias.has_value() && decay_mode == FRWKV_DECAY_RAW_W),
              "decay_bias is only defined for decay logits");
  c10::DeviceGuard guard(state.device());
  Prepared launch;
  if (validated_metadata.has_value() && validated_metadata->defined()) {
    (*validated_metadata)->check_compatible(query_start_loc, state_indices, r.size(0),
                                            state.size(0), -1);
    launch = (*validated_metadata)->prepared();
  } else {
    launch = device_prepare(query_start_loc, state_indices, r.size(0), state.size(0));
  }
  check_rc(frwkv_recurrent_tmix_fused_forward(
      io_code(r.scalar_type()), static_cast<int>(decay_mode),
      static_cast<int32_t>(state_indices.numel()), static_cast<int32_t>(state.size(1)), 64,
      static_cast<int32_t>(r.size(0)), static_cast<int32_t>(state.size(0)),
      launch.cu_snapshot.data_ptr<int32_t>(), launch.slot_snapshot.data_ptr<int32_t>(),
      launch.status.data_ptr<int32_t>(), state.data_ptr<float>(), r.data_ptr(),
      decay.data_ptr(), decay_bias.has_value() ? decay_bias->data_ptr() : nullptr, k.data_ptr(),
      v.data_ptr(), a12.data_ptr(), g.data_ptr(), k_k.data_ptr(), a0.data_ptr(), k_a.data_ptr(),
      r_k.data_ptr(), ln_weight.data_ptr(), ln_bias.data_ptr(), output.data_ptr(),
      static_cast<float>(scale), current_stream(state)));
  return output;
}

TORCH_LIBRARY(flashrwkv2, m) {
  m.class_<MetadataTicket>("MetadataTicket")
      .def("max_seqlen", [](const TicketPtr& t) { return t->max_seqlen(); })
      .def("total_tokens", [](const TicketPtr& t) { return t->total_tokens(); })
      .def("state_pool_size", [](const TicketPtr& t) { return t->state_pool_size(); })
      .def("status", [](const TicketPtr& t) { return t->prepared().status; })
      .def("query_start_loc_snapshot",
           [](const TicketPtr& t) { return t->prepared().cu_snapshot; })
      .def("state_indices_snapshot",
           [](const TicketPtr& t) { return t->prepared().slot_snapshot; })
      .def("check_compatible",
           [](const TicketPtr& t, Tensor cu, Tensor slots, int64_t total_tokens,
              int64_t state_pool_size, int64_t max_seqlen) {
             t->check_compatible(cu, slots, total_tokens, state_pool_size, max_seqlen);
           })
      // The reference ticket's method names
      // (infer_recurrent_fp32io16_forward_varlen.cpp:314-345).
      .def("_check_compatible",
           [](const TicketPtr& t, Tensor cu, Tensor slots, int64_t total_tokens,
              int64_t state_pool_size, int64_t max_seqlen) {
             t->check_compatible(cu, slots, total_tokens, state_pool_size, max_seqlen);
           })
      .def("_query_start_loc_snapshot",
           [](const TicketPtr& t) { return t->prepared().cu_snapshot; })
      .def("_state_indices_snapshot",
           [](const TicketPtr& t) { return t->prepared().slot_snapshot; })
      .def("_status", [](const TicketPtr& t) { return t->prepared().status; })
      .def("_max_seqlen", [](const TicketPtr& t) { return t->max_seqlen(); });
  m.def(
      "prepare_recurrent_metadata(Tensor query_start_loc, Tensor state_indices, "
      "int total_tokens, int state_pool_size, int max_seqlen=-1) -> "
      "__torch__.torch.classes.flashrwkv2.MetadataTicket",
      &prepare_recurrent_metadata);
  m.def(
      "recurrent_fp32_from_decay_logits(Tensor query_start_loc, Tensor "
      "state_indices, Tensor(a!) state, Tensor r, Tensor decay_logits, Tensor k, "
      "Tensor v, Tensor a, Tensor b, Tensor(b!) output, float scale, "
      "Tensor? decay_bias=None, "
      "__torch__.torch.classes.flashrwkv2.MetadataTicket? "
      "validated_metadata=None, int max_seqlen=-1) -> ()",
      &recurrent_fp32_from_decay_logits);
  m.def(
      "recurrent_fp32_forward_internal(Tensor query_start_loc, Tensor "
      "state_indices, Tensor(a!) state, Tensor r, Tensor decay, Tensor k, "
      "Tensor v, Tensor a, Tensor b, Tensor(b!) output, float scale, "
      "int decay_mode, Tensor? decay_bias=None, "
      "__torch__.torch.classes.flashrwkv2.MetadataTicket? "
      "validated_metadata=None, int max_seqlen=-1) -> ()",
      &recurrent_fp32_forward_internal);
  m.def(
      "pretrain_tmix_lnx_rkvres_xg_forward(Tensor x, Tensor r, Tensor k, Tensor v, "
      "Tensor residual_scale, Tensor weight, Tensor bias, Tensor g, int head_size=64) -> "
      "(Tensor, Tensor, Tensor)",
      &pretrain_tmix_lnx_rkvres_xg_forward);
  m.def(
      "pretrain_tmix_lnx_rkvres_xg_backward(Tensor grad_output, Tensor x, Tensor r, Tensor k, "
      "Tensor v, Tensor residual_scale, Tensor weight, Tensor bias, Tensor g, Tensor mean, "
      "Tensor rstd, int head_size=64) -> Tensor[]",
      &pretrain_tmix_lnx_rkvres_xg_backward);
  m.def("set_recurrent_long_route(int route) -> int", &set_recurrent_long_route);
  m.def("recurrent_long_route() -> int", &recurrent_long_route);
  m.def(
      "infer_chunk_bf16_forward_varlen(Tensor r, Tensor decay_logits, Tensor k, "
      "Tensor v, Tensor a, Tensor b, Tensor(a!) state_pool, Tensor cu_seqlens, "
      "Tensor state_indices, int chunk_size=16, int max_seqlen=-1, float scale=1.0, "
      "Tensor? decay_bias=None) -> (Tensor, Tensor(a!))",
      &infer_chunk_bf16_forward_varlen);
  m.def(
      "chunk_forward_internal(Tensor r, Tensor decay, Tensor k, Tensor v, Tensor a, "
      "Tensor b, Tensor(a!) state_pool, Tensor cu_seqlens, Tensor state_indices, "
      "float scale, int decay_mode, Tensor? decay_bias=None) -> Tensor",
      &chunk_forward_internal);
  m.def(
      "statetune_recurrent_fp32io16_forward(Tensor sequence_chunk_offsets, "
      "Tensor chunk_token_starts, Tensor chunk_token_ends, Tensor(a!) state, Tensor r, "
      "Tensor decay_logits, Tensor k, Tensor v, Tensor a, Tensor b, Tensor(b!) output, "
      "Tensor(c!) boundary, Tensor(d!) state_dot_a, float scale=1.0) -> ()",
      &statetune_recurrent_fp32io16_forward);
  m.def(
      "statetune_forward_internal(Tensor sequence_chunk_offsets, "
      "Tensor chunk_token_starts, Tensor chunk_token_ends, Tensor(a!) state, Tensor r, "
      "Tensor decay, Tensor k, Tensor v, Tensor a, Tensor b, Tensor(b!) output, "
      "Tensor(c!) boundary, Tensor(d!) state_dot_a, Tensor(e!)? interior, float scale, "
      "int decay_mode) -> ()",
      &statetune_forward_internal);
  m.def(
      "statetune_recurrent_fp32io16_backward(Tensor sequence_chunk_offsets, "
      "Tensor chunk_token_starts, Tensor chunk_token_ends, Tensor final_state, Tensor r, "
      "Tensor decay_logits, Tensor k, Tensor v, Tensor a, Tensor b, Tensor state_dot_a, "
      "Tensor? grad_output, Tensor? grad_final_state, Tensor boundary, "
      "Tensor(a!)? grad_r, Tensor(b!)? grad_decay_logits, Tensor(c!)? grad_k, "
      "Tensor(d!)? grad_v, Tensor(e!)? grad_a, Tensor(f!)? grad_b, "
      "Tensor(g!)? grad_initial_state, float scale=1.0) -> ()",
      &statetune_recurrent_fp32io16_backward);
  m.def(
      "statetune_backward_internal(Tensor sequence_chunk_offsets, Tensor chunk_token_starts, "
      "Tensor chunk_token_ends, Tensor r, Tensor decay, Tensor k, Tensor v, Tensor a, "
      "Tensor b, Tensor? grad_output, Tensor? grad_final_state, Tensor boundary, "
      "Tensor(a!) grad_r, Tensor(b!) grad_decay, Tensor(c!) grad_k, Tensor(d!) grad_v, "
      "Tensor(e!) grad_a, Tensor(f!) grad_b, Tensor(g!) grad_initial_state, "
      "Tensor? interior, float scale, int decay_mode) -> ()",
      &statetune_backward_internal);
  m.def(
      "rl_infctx_chunk_fp32io16_forward(Tensor sequence_chunk_offsets, Tensor chunk_token_starts, "
      "Tensor chunk_token_ends, Tensor state, Tensor r, Tensor decay_logits, Tensor k, "
      "Tensor v, Tensor a, Tensor b, int strategy=1, float scale=1.0, "
      "Tensor? decay_bias=None) -> (Tensor, Tensor)",
      &rl_infctx_forward);
  m.def(
      "rl_infctx_chunk_fp32io16_backward_replay(Tensor chunk_token_starts, "
      "Tensor chunk_token_ends, Tensor boundary, Tensor r, Tensor decay_logits, Tensor k, "
      "Tensor v, Tensor a, Tensor b, Tensor(a!) output, Tensor(b!) state_dot_a, "
      "float scale=1.0, Tensor? decay_bias=None) -> ()",
      &rl_infctx_replay);
  m.def(
      "recurrent_fp16_from_decay_logits(Tensor query_start_loc, Tensor state_indices, "
      "Tensor elapsed_state_pool, Tensor(a!) state, Tensor r, Tensor decay_logits, "
      "Tensor k, Tensor v, Tensor a, Tensor b, Tensor(b!) output, float scale, "
      "Tensor? decay_bias=None, "
      "__torch__.torch.classes.flashrwkv2.MetadataTicket? "
      "validated_metadata=None, int max_seqlen=-1) -> ()",
      &recurrent_fp16_from_decay_logits);
  m.def("recurrent_fp16_advance_i32(Tensor(a!) elapsed_state, int amount) -> ()",
        &recurrent_fp16_advance_i32);
  m.def(
      "recurrent_fp16_advance_i32_varlen(Tensor query_start_loc, Tensor state_indices, "
      "Tensor(a!) elapsed_state_pool, int total_tokens, "
      "__torch__.torch.classes.flashrwkv2.MetadataTicket? "
      "validated_metadata=None) -> ()",
      &recurrent_fp16_advance_i32_varlen);
  m.def("recurrent_add_vec_forward_varlen(Tensor x, Tensor vec) -> Tensor",
        &recurrent_add_vec_forward_varlen);
  m.def(
      "tmix_kk_a_gate_forward_varlen(Tensor k, Tensor k_k, Tensor a0, Tensor a12, Tensor k_a, "
      "int head_size=64, int batch_size=1, int max_seqlen=1) -> (Tensor, Tensor, Tensor)",
      &tmix_kk_a_gate_forward_varlen);
  m.def(
      "tmix_lnx_rkvres_xg_forward_varlen(Tensor x, Tensor r, Tensor k, Tensor v, Tensor r_k, "
      "Tensor weight, Tensor bias, Tensor g, int head_size=64, int batch_size=1, "
      "int max_seqlen=1) -> Tensor",
      &tmix_lnx_rkvres_xg_forward_varlen);
  m.def(
      "recurrent_tmix_fused_forward(Tensor query_start_loc, Tensor state_indices, "
      "Tensor(a!) state, Tensor r, Tensor decay, Tensor k, Tensor v, Tensor a12, Tensor g, "
      "Tensor k_k, Tensor a0, Tensor k_a, Tensor r_k, Tensor ln_weight, Tensor ln_bias, "
      "float scale=1.0, int decay_mode=0, Tensor? decay_bias=None, "
      "__torch__.torch.classes.flashrwkv2.MetadataTicket? validated_metadata=None) -> Tensor",
      &recurrent_tmix_fused_forward);
}

// The reference's pretraining operator namespace (pretrain_recurrent_bf16_forward.cpp:50-53).
TORCH_LIBRARY(rwkv7_clampw_v3, m) {
  m.def(
      "forward(Tensor r, Tensor w, Tensor k, Tensor v, Tensor a, Tensor b, Tensor(a!) y, "
      "Tensor(b!) s, Tensor(c!) sa, int head_size) -> ()",
      &clampw_forward);
  m.def(
      "backward(Tensor r, Tensor w, Tensor k, Tensor v, Tensor a, Tensor b, Tensor dy, "
      "Tensor s, Tensor sa, Tensor(a!) dr, Tensor(b!) dw, Tensor(c!) dk, Tensor(d!) dv, "
      "Tensor(e!) da, Tensor(f!) db, int head_size) -> ()",
      &clampw_backward);
}

#ifdef FRWKV_PYTHON_MODULE
// Direct Python entry points for the per-token decode chain, in the
// reference's binding style (a pybind11 module, csrc/registration.cpp:6-8).
// A call converts its arguments once and runs the same function as the
// TORCH_LIBRARY op above (same checks, same errors); it skips the
// dispatcher's boxed path, which costs several microseconds per call at
// these ops' 10-19 arguments. The ticket arrives as the custom class's
// Python object and is unwrapped to the same intrusive pointer.
#include <torch/csrc/jit/python/pybind_utils.h>
#include <torch/extension.h>

namespace {

std::optional<TicketPtr> ticket_arg(const pybind11::object& obj) {
  if (obj.is_none()) return std::nullopt;
  c10::IValue value;
  try {
    value = torch::jit::toIValue(obj, c10::getCustomClassType<TicketPtr>());
  } catch (const std::exception&) {
    TORCH_CHECK(false, "validated_metadata must be None or a ticket returned by "
                "prepare_recurrent_metadata, got ",
                pybind11::str(pybind11::type::of(obj).attr("__name__")).cast<std::string>());
  }
  return value.toCustomClass<MetadataTicket>();
}

}  // namespace

PYBIND11_MODULE(_flashrwkv_amd_ops, m) {
  namespace py = pybind11;
  // TORCH_CHECK failures surface as RuntimeError with the check's message,
  // as they do through the ops (no C++ backtrace).
  py::register_local_exception_translator([](std::exception_ptr error) {
    try {
      if (error) std::rethrow_exception(error);
    } catch (const c10::Error& e) {
      PyErr_SetString(PyExc_RuntimeError, e.what_without_backtrace());
    }
  });
  m.def("recurrent_fp32_from_decay_logits",
        [](Tensor cu, Tensor slots, Tensor state, Tensor r, Tensor x, Tensor k, Tensor v,
           Tensor a, Tensor b, Tensor out, double scale, std::optional<Tensor> bias,
           py::object ticket, int64_t max_seqlen) {
          recurrent_fp32_from_decay_logits(cu, slots, state, r, x, k, v, a, b, out, scale,
                                           bias, ticket_arg(ticket), max_seqlen);
        });
  m.def("recurrent_fp32_forward_internal",
        [](Tensor cu, Tensor slots, Tensor state, Tensor r, Tensor x, Tensor k, Tensor v,
           Tensor a, Tensor b, Tensor out, double scale, int64_t decay_mode,
           std::optional<Tensor> bias, py::object ticket, int64_t max_seqlen) {
          recurrent_fp32_forward_internal(cu, slots, state, r, x, k, v, a, b, out, scale,
                                          decay_mode, bias, ticket_arg(ticket), max_seqlen);
        });
  m.def("recurrent_fp16_from_decay_logits",
        [](Tensor cu, Tensor slots, Tensor elapsed, Tensor state, Tensor r, Tensor x, Tensor k,
           Tensor v, Tensor a, Tensor b, Tensor out, double scale, std::optional<Tensor> bias,
           py::object ticket, int64_t max_seqlen) {
          recurrent_fp16_from_decay_logits(cu, slots, elapsed, state, r, x, k, v, a, b, out,
                                           scale, bias, ticket_arg(ticket), max_seqlen);
        });
  m.def("recurrent_fp16_advance_i32", &recurrent_fp16_advance_i32);
  m.def("recurrent_fp16_advance_i32_varlen",
        [](Tensor cu, Tensor slots, Tensor elapsed, int64_t total_tokens, py::object ticket) {
          recurrent_fp16_advance_i32_varlen(cu, slots, elapsed, total_tokens,
                                            ticket_arg(ticket));
        });
  m.def("recurrent_add_vec_forward_varlen", &recurrent_add_vec_forward_varlen);
  m.def("tmix_kk_a_gate_forward_varlen", &tmix_kk_a_gate_forward_varlen);
  m.def("tmix_lnx_rkvres_xg_forward_varlen", &tmix_lnx_rkvres_xg_forward_varlen);
  m.def("recurrent_tmix_fused_forward",
        [](Tensor cu, Tensor slots, Tensor state, Tensor r, Tensor decay, Tensor k, Tensor v,
           Tensor a12, Tensor g, Tensor k_k, Tensor a0, Tensor k_a, Tensor r_k,
           Tensor ln_weight, Tensor ln_bias, double scale, int64_t decay_mode,
           std::optional<Tensor> bias, py::object ticket) {
          return recurrent_tmix_fused_forward(cu, slots, state, r, decay, k, v, a12, g, k_k,
                                              a0, k_a, r_k, ln_weight, ln_bias, scale,
                                              decay_mode, bias, ticket_arg(ticket));
        });
}
#endif  // FRWKV_PYTHON_MODULE

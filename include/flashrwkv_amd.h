/*
 * flashrwkv_amd -- C ABI of the MI355X-native WKV7 operator family.
 *
 * libflashrwkv_amd.so exports these entry points. They take plain device
 * pointers, sizes and a HIP stream (passed as void*, a hipStream_t; NULL is
 * the null stream), launch hand-written gfx950 HIP kernels on that stream and
 * return immediately: no host synchronisation and no device allocation (entry
 * points that need scratch memory take a caller workspace, sized by a
 * matching *_bytes query). Every call returns FRWKV_OK or an error code;
 * frwkv_last_error() gives the message of the last failing call on the
 * calling thread.
 *
 * Tensor conventions (all row-major, contiguous, device memory):
 *   tokens   r, decay, k, v, a, b, output: [total_tokens, H, D] of io_dtype
 *   state    pool [slots, H, D, D] laid out [K,V] (state[slot][h][key][value])
 *   metadata cu_seqlens int32 [B+1], state_indices int32 [B]
 *   decay    FRWKV_DECAY_LOGITS: raw decay logits x, retention
 *            w = exp(-e^{-1/2} sigmoid(x + bias)) (the reference boundary);
 *            FRWKV_DECAY_RAW_W: the retention w itself (bias must be NULL).
 *   recurrence per token: sa = S^T a; S = diag(w) S + b sa^T + k v^T;
 *            y = scale S^T r.
 *   The chunked (head size 64) kernels take at most 65536 heads; a call
 *   routed to them with more returns FRWKV_ERR_UNSUPPORTED.
 *
 * Each entry point cites the reference native interface it replaces
 * (paths relative to the rwkv-rs/FlashRWKV2 source tree).
 */
#ifndef FLASHRWKV_AMD_H_
#define FLASHRWKV_AMD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FRWKV_ABI_VERSION 2

enum frwkv_status {
  FRWKV_OK = 0,
  FRWKV_ERR_INVALID_ARGUMENT = 1,
  FRWKV_ERR_UNSUPPORTED = 2,
  FRWKV_ERR_HIP = 3
};

enum frwkv_dtype {
  FRWKV_DTYPE_F32 = 0,
  FRWKV_DTYPE_F16 = 1,
  FRWKV_DTYPE_BF16 = 2
};

enum frwkv_decay_mode {
  FRWKV_DECAY_LOGITS = 0,
  FRWKV_DECAY_RAW_W = 1
};

/* Metadata status bits written by frwkv_metadata_validate (same bit meanings
 * as csrc/validation/recurrent_metadata.cu:15-20). */
enum frwkv_metadata_error {
  FRWKV_META_BAD_ENDPOINT = 1,
  FRWKV_META_BAD_RANGE = 2,
  FRWKV_META_BAD_SLOT = 4,
  FRWKV_META_DUPLICATE_SLOT = 8
};

/* ABI version of the loaded library (FRWKV_ABI_VERSION at build time). */
int frwkv_abi_version(void);

/* Static description of a status code. */
const char* frwkv_status_string(int status);

/* Message of the last failing call on this thread ("" if none). */
const char* frwkv_last_error(void);

/*
 * Validates packed metadata on the device and snapshots it.
 * Replaces prepare_recurrent_metadata_cuda / validate_recurrent_metadata_kernel
 * (csrc/validation/recurrent_metadata.cu:22-97, 99-140).
 * Writes status[0] = OR of frwkv_metadata_error bits (0 when valid) and copies
 * cu_seqlens / state_indices into the snapshots, which later launches read so
 * that a caller mutating its metadata afterwards cannot change a launch.
 * Requires 1 <= num_sequences <= 65535, total_tokens > 0, state_pool_size > 0.
 */
int frwkv_metadata_validate(const int32_t* cu_seqlens,
                            const int32_t* state_indices,
                            int32_t num_sequences, int32_t total_tokens,
                            int32_t state_pool_size, int32_t* status,
                            int32_t* cu_seqlens_snapshot,
                            int32_t* state_indices_snapshot, void* stream);

/*
 * fp32-state recurrent forward over packed varlen sequences, state pool
 * updated in place at state_indices.
 * Replaces recurrent_fp32_from_decay_logits_cuda
 * (csrc/sm120/tmix/wkv7/infer_recurrent_fp32io16_forward_varlen.cu:448-508).
 * head_size in {64, 128, 256}; io_dtype F16/BF16/F32; decay_bias NULL or
 * [H*D] of io_dtype (logits mode only). metadata_status is the status word of
 * frwkv_metadata_validate: when it is non-zero at run time the kernels fill
 * output with NaN and leave the pool untouched. max_seqlen is the longest
 * sequence (<= 0: unknown). It selects the kernel:
 *   - unknown, or below 64, or tokens other than bf16, or head size other
 *     than 64: the per-token kernel, fp32 arithmetic per token (one wave per
 *     state for decode, four for longer sequences);
 *   - bf16 tokens, head size 64, max_seqlen >= 64: the chunked form on
 *     split-bf16 MFMA products (about 2^-17 relative error per split
 *     operand). Outputs and states then stay within the reference's
 *     relative-RMSE gate for this operator (0.002, reference
 *     tests/fixtures/tolerances-v1.json:9-12), at several times the speed.
 */
int frwkv_recurrent_forward(int io_dtype, int decay_mode, int32_t num_sequences,
                            int32_t num_heads, int32_t head_size,
                            int32_t total_tokens, int32_t max_seqlen,
                            int32_t state_pool_size, const int32_t* cu_seqlens,
                            const int32_t* state_indices,
                            const int32_t* metadata_status, float* state_pool,
                            const void* r, const void* decay,
                            const void* decay_bias, const void* k,
                            const void* v, const void* a, const void* b,
                            void* output, float scale, void* stream);

/*
 * fp16-state recurrent forward (the Albatross family), pool [slots,H,D,D] of
 * fp16 updated in place at state_indices.
 * Replaces recurrent_fp16_from_decay_logits_cuda and its dispatch
 * (csrc/sm120/tmix/wkv7/infer_recurrent_fp16_forward_varlen.cu:1078-1215,
 * 1283-1365; binding .cpp:210-270). Tokens, decay_bias and output are fp16;
 * the decay is given as logits. Per token, with phase = elapsed_state_pool
 * [slot] + h*D + key + (t - sequence start), dither(p) = 2^-41 *
 * int32(p * 2654435769 mod 2^32) and delta = fp16(w - 1 + dither):
 *   sa = S^T a; S = fp16(S + diag(delta) S + b sa^T + k v^T);
 *   y = fp16(scale S^T r)
 * with fp32 arithmetic between the roundings. elapsed_state_pool [slots]
 * int32 is read, not advanced (frwkv_advance_i32_varlen advances it).
 * head_size in {64, 128, 256}; metadata_status and max_seqlen as for
 * frwkv_recurrent_forward.
 */
int frwkv_recurrent_fp16_forward(int32_t num_sequences, int32_t num_heads,
                                 int32_t head_size, int32_t total_tokens,
                                 int32_t max_seqlen, int32_t state_pool_size,
                                 const int32_t* cu_seqlens, const int32_t* state_indices,
                                 const int32_t* metadata_status,
                                 const int32_t* elapsed_state_pool, void* state_pool,
                                 const void* r, const void* decay_logits,
                                 const void* decay_bias, const void* k, const void* v,
                                 const void* a, const void* b, void* output, float scale,
                                 void* stream);

/*
 * elapsed_state[i] += amount for i < count (int32, wrapping).
 * Replaces recurrent_fp16_advance_i32_cuda
 * (csrc/sm120/tmix/wkv7/infer_recurrent_fp16_forward_varlen.cu:57-64, 1217-1228).
 */
int frwkv_advance_i32(int32_t* elapsed_state, int64_t count, int32_t amount, void* stream);

/*
 * elapsed_state_pool[state_indices[s]] += cu_seqlens[s+1] - cu_seqlens[s] for
 * every sequence s; nothing when metadata_status[0] != 0 at run time.
 * Replaces recurrent_fp16_advance_i32_varlen_cuda
 * (csrc/sm120/tmix/wkv7/infer_recurrent_fp16_forward_varlen.cu:67-81, 1230-1245).
 */
int frwkv_advance_i32_varlen(int32_t num_sequences, int32_t state_pool_size,
                             const int32_t* cu_seqlens, const int32_t* state_indices,
                             const int32_t* metadata_status, int32_t* elapsed_state_pool,
                             void* stream);

/*
 * output[n,c] = fp16(float(x[n,c]) + float(vec[c])) for x [rows,channels]
 * fp16 (channels even; x, vec, output 4-byte aligned).
 * Replaces recurrent_add_vec_forward_varlen_cuda
 * (csrc/sm120/tmix/wkv7/infer_recurrent_fp16_forward_varlen.cu:85-122, 1247-1281).
 */
int frwkv_add_vec(int64_t rows, int32_t channels, const void* x, const void* vec,
                  void* output, void* stream);

/*
 * Chunked forward over packed varlen sequences (prefill), state pool updated
 * in place at state_indices. Exact chunk form of the recurrence on bf16 MFMA
 * with fp32 accumulation and an fp32 state carried between 64-token chunks;
 * results equal frwkv_recurrent_forward up to bf16 rounding.
 * Replaces infer_chunk_bf16_forward_varlen_cuda and its K1/K2 kernels
 * (csrc/sm120/tmix/wkv7/infer_chunk_bf16_forward_varlen.cu:42-334; binding
 * infer_chunk_bf16_forward_varlen.cpp:77-171), whose chunk_size argument has
 * no counterpart here: the result does not depend on the chunking.
 * head_size must be 64; io_dtype F16/BF16; pool_dtype F32 (fp32 pool) or
 * BF16 (the reference contract's bf16 pool, read and written as bf16);
 * metadata_status as in frwkv_recurrent_forward (non-zero: NaN output, pool
 * untouched). In FRWKV_DECAY_RAW_W mode the retention is clamped to
 * [2^-20, 1].
 */
int frwkv_chunk_forward(int io_dtype, int decay_mode, int pool_dtype,
                        int32_t num_sequences, int32_t num_heads,
                        int32_t head_size, int32_t total_tokens,
                        int32_t state_pool_size, const int32_t* cu_seqlens,
                        const int32_t* state_indices,
                        const int32_t* metadata_status, void* state_pool,
                        const void* r, const void* decay,
                        const void* decay_bias, const void* k, const void* v,
                        const void* a, const void* b, void* output, float scale,
                        void* stream);

/*
 * Training (StateTune) forward with caller chunk metadata: sequence s owns
 * chunks sequence_chunk_offsets[s] .. sequence_chunk_offsets[s+1]-1, chunk c
 * covers tokens chunk_token_starts[c] .. chunk_token_ends[c]-1 (any length;
 * a range reaching outside [0, total_tokens) is clamped to it, and an end
 * before the start makes the chunk empty; the backward reads the metadata
 * the same way).
 * state [B,H,D,D] fp32 holds S0 on entry and the final state on return (the
 * caller passes a copy). boundary [num_chunks,H,D,D] fp32 receives the state
 * at each chunk start; state_dot_a [total_tokens,H,D] fp32 receives
 * a_t^T S_{t-1}. interior (NULL: not written) receives the state at every
 * piece start inside a chunk, at slot (piece start) / P, where the piece
 * length P is 64 tokens for head size 64 and 16 for 128 and 256; it holds
 * frwkv_statetune_interior_bytes, and only the slots of chunks longer than P
 * are written. Interior piece starts of different chunks lie more than P
 * tokens apart, so the slots never collide. The buffer is opaque to the
 * caller: [D,D] fp32 per (slot, head) at head sizes 64 and 256; at 128 the
 * states rounded to bf16 in the kernels' own element order (the backward
 * uses a piece's start state only as bf16 MFMA operands).
 * Replaces statetune_recurrent_fp32io16_forward_cuda
 * (csrc/sm90/tmix/wkv7/statetune_recurrent_fp32io16_forward.cu:32-224;
 * binding statetune_recurrent_fp32io16_forward.cpp:26-56). head_size 64
 * runs the chunked MFMA kernel, 128 the MFMA kernel over 16-token pieces,
 * 256 the per-token fp32 kernel.
 */
int frwkv_statetune_forward(int io_dtype, int decay_mode, int32_t num_sequences,
                            int32_t num_heads, int32_t head_size,
                            int32_t total_tokens, int32_t num_chunks,
                            const int32_t* sequence_chunk_offsets,
                            const int32_t* chunk_token_starts,
                            const int32_t* chunk_token_ends, float* state,
                            const void* r, const void* decay,
                            const void* decay_bias, const void* k,
                            const void* v, const void* a, const void* b,
                            void* output, float* boundary, float* state_dot_a,
                            float* interior, float scale, void* stream);

/* Bytes of the interior-state buffer of frwkv_statetune_forward /
 * frwkv_statetune_backward: ceil(total_tokens / P) x H x D x D elements of
 * 4 bytes (fp32; 2 bytes, bf16, at head size 128). */
size_t frwkv_statetune_interior_bytes(int32_t head_size, int32_t num_heads,
                                      int32_t total_tokens);

/*
 * The interior states of frwkv_statetune_forward, recomputed from the chunk
 * start states boundary [num_chunks,H,D,D] (read only): for every chunk longer
 * than the piece length P, the state at each of its interior piece starts
 * goes to interior at slot (piece start) / P. Chunks of at most P tokens are
 * skipped, and no output is written. No counterpart in the reference, whose
 * backward rebuilds states by dividing by the decay; for callers of the
 * backward that did not keep the forward's interior states.
 */
int frwkv_statetune_interior(int io_dtype, int decay_mode, int32_t num_heads,
                             int32_t head_size, int32_t total_tokens,
                             int32_t num_chunks, const int32_t* chunk_token_starts,
                             const int32_t* chunk_token_ends, const float* boundary,
                             const void* r, const void* decay, const void* decay_bias,
                             const void* k, const void* v, const void* a,
                             const void* b, float* interior, void* stream);

/*
 * Training (StateTune) backward. Recomputes every piece's forward quantities
 * from its start state -- boundary (the state at each chunk start) for a
 * chunk's first piece, interior for the others -- and runs the chunked
 * adjoint in reverse; it never divides by the decay, and any chunk length
 * and any retention are supported (pieces whose decay span exceeds the
 * kernel's single-reference limit run as 16- and 4-token sub-pieces).
 * interior: the forward's interior states, or NULL; then the call first
 * recomputes them into the workspace (frwkv_statetune_interior), which must
 * be given (FRWKV_ERR_INVALID_ARGUMENT otherwise, before anything runs).
 * grad_output [total_tokens,H,D] (io dtype) and
 * grad_final_state [B,H,D,D] fp32 may be NULL (zero). Writes every token
 * gradient (grad_decay is dL/d(decay input): logits or retention per
 * decay_mode) and grad_initial_state [B,H,D,D] fp32.
 * workspace: frwkv_statetune_backward_workspace_bytes(head_size, H,
 * total_tokens, interior != NULL) bytes of device memory, 256-byte aligned;
 * it may be NULL only when that is 0 (head sizes 64 and 128 with interior
 * given).
 * Replaces statetune_recurrent_fp32io16_backward_cuda
 * (csrc/sm90/tmix/wkv7/statetune_recurrent_fp32io16_backward.cu:49-676;
 * binding statetune_recurrent_fp32io16_backward.cpp:34-82). head_size 64
 * runs the chunked MFMA kernel, 128 the MFMA kernel over 16-token pieces, 256
 * the per-token fp32 kernel (with fp32 gradient slices in the workspace, added
 * in a fixed order).
 */
int frwkv_statetune_backward(int io_dtype, int decay_mode, int32_t num_sequences,
                             int32_t num_heads, int32_t head_size,
                             int32_t total_tokens, int32_t num_chunks,
                             const int32_t* sequence_chunk_offsets,
                             const int32_t* chunk_token_starts,
                             const int32_t* chunk_token_ends,
                             const float* boundary, const float* interior,
                             const void* r, const void* decay, const void* decay_bias,
                             const void* k, const void* v, const void* a,
                             const void* b, const void* grad_output,
                             const float* grad_final_state, void* grad_r,
                             void* grad_decay, void* grad_k, void* grad_v,
                             void* grad_a, void* grad_b,
                             float* grad_initial_state, void* workspace,
                             size_t workspace_bytes, float scale, void* stream);

/* Workspace bytes of frwkv_statetune_backward (0: none needed). */
size_t frwkv_statetune_backward_workspace_bytes(int32_t head_size, int32_t num_heads,
                                                int32_t total_tokens, int interior_given);

/* Size of the per-device static scratch of frwkv_statetune_backward_noalloc. */
#define FRWKV_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)

/*
 * frwkv_statetune_backward without the workspace argument: the workspace
 * (frwkv_statetune_backward_workspace_bytes(head_size, H, total_tokens,
 * interior != NULL) bytes) lives in a static device array of
 * FRWKV_NOALLOC_SCRATCH_BYTES (64 MiB), in a code object of its own that a
 * device loads at this entry's first call on it and holds until the process
 * ends (a process that never calls it holds none of it); larger needs are
 * rejected with FRWKV_ERR_INVALID_ARGUMENT before anything runs. The call
 * allocates and frees nothing. Every call on one device shares that device's
 * array: calls that overlap on one device (other streams, other threads)
 * race and must be serialised by the caller. Outputs and every other
 * argument as frwkv_statetune_backward (the same kernels run).
 * No counterpart in the reference; for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving or training loops,
 * harnesses that forbid hipMalloc).
 */
int frwkv_statetune_backward_noalloc(int io_dtype, int decay_mode, int32_t num_sequences,
                                     int32_t num_heads, int32_t head_size,
                                     int32_t total_tokens, int32_t num_chunks,
                                     const int32_t* sequence_chunk_offsets,
                                     const int32_t* chunk_token_starts,
                                     const int32_t* chunk_token_ends,
                                     const float* boundary, const float* interior,
                                     const void* r, const void* decay,
                                     const void* decay_bias, const void* k,
                                     const void* v, const void* a, const void* b,
                                     const void* grad_output,
                                     const float* grad_final_state, void* grad_r,
                                     void* grad_decay, void* grad_k, void* grad_v,
                                     void* grad_a, void* grad_b,
                                     float* grad_initial_state, float scale,
                                     void* stream);

/*
 * Pretraining forward (clampw v3): dense tokens [B,T,H,D] (token t of
 * sequence s at row s*T + t), S0 = 0, no final state. boundary
 * [B,H,T/16,D,D] fp32 receives the state every 16 tokens (entry i: the state
 * before token 16 i); state_dot_a [B,T,H,D] fp32 receives a_t^T S_{t-1}.
 * T must be a multiple of 16; head_size 64, 128 or 256 (64 on the chunked
 * MFMA kernel, 128 on the MFMA piece kernel, 256 on the per-token fp32
 * kernel).
 * Replaces rwkv7_clampw_v3::forward / cuda_forward_v3
 * (csrc/sm90/tmix/wkv7/pretrain_recurrent_bf16_forward.cpp:20-26, 50-53;
 * kernel pretrain_recurrent_bf16_forward.cu).
 */
int frwkv_pretrain_forward(int io_dtype, int decay_mode, int32_t batch, int32_t tokens,
                           int32_t num_heads, int32_t head_size, const void* r,
                           const void* decay, const void* k, const void* v,
                           const void* a, const void* b, void* output, float* boundary,
                           float* state_dot_a, void* stream);

/*
 * Pretraining backward: recomputes every chunk from the boundary written by
 * frwkv_pretrain_forward (head size 64: 64-token chunks from every 4th entry;
 * 128 and 256: every 16-token entry) and writes the six token gradients
 * (grad_decay is dL/d(decay input)). grad_output may not be NULL. workspace:
 * frwkv_pretrain_backward_workspace_bytes of device memory (head size 256:
 * fp32 gradient slices; else 0, and workspace may be NULL).
 * Replaces rwkv7_clampw_v3::backward / cuda_backward_v3
 * (csrc/sm90/tmix/wkv7/pretrain_recurrent_bf16_forward.cpp:31-53).
 */
int frwkv_pretrain_backward(int io_dtype, int decay_mode, int32_t batch, int32_t tokens,
                            int32_t num_heads, int32_t head_size, const void* r,
                            const void* decay, const void* k, const void* v,
                            const void* a, const void* b, const void* grad_output,
                            const float* boundary, void* grad_r, void* grad_decay,
                            void* grad_k, void* grad_v, void* grad_a, void* grad_b,
                            void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes of frwkv_pretrain_backward (0: none needed). */
size_t frwkv_pretrain_backward_workspace_bytes(int32_t batch, int32_t tokens,
                                               int32_t num_heads, int32_t head_size);

/*
 * Replay stage of the RL/infctx chunk family: chunk c runs tokens
 * chunk_token_starts[c] .. chunk_token_ends[c]-1 starting from boundary[c]
 * ([num_chunks,H,D,D] fp32, read only) and writes output [total_tokens,H,D]
 * (io dtype) and state_dot_a [total_tokens,H,D] fp32 (a_t^T S_{t-1}) for
 * those tokens. head_size 64 runs the chunked bf16-MFMA kernel, 128 and 256
 * the fp32 per-token kernel. decay_bias NULL or [H*D] (logits mode only).
 * Replaces rl_infctx_chunk_fp32io16_backward_replay
 * (csrc/sm90/rl_infctx/wkv7/rl_infctx_chunk_fp32io16_backward.cpp:102-124).
 * The RL/infctx forward (rl_infctx_chunk_fp32io16_forward.cpp:157-229) needs
 * no entry of its own: it is frwkv_chunk_forward (head size 64) or
 * frwkv_recurrent_forward (128, 256) on a working copy of the gathered pool.
 */
int frwkv_chunk_replay(int io_dtype, int decay_mode, int32_t num_chunks, int32_t num_heads,
                       int32_t head_size, int32_t total_tokens,
                       const int32_t* chunk_token_starts, const int32_t* chunk_token_ends,
                       const float* boundary, const void* r, const void* decay,
                       const void* decay_bias, const void* k, const void* v, const void* a,
                       const void* b, void* output, float* state_dot_a, float scale,
                       void* stream);

/*
 * TMix producer of the WKV7 inputs, per (token, head) row of head_size
 * features of packed k, a12 [total_tokens, H*head_size] with per-channel
 * k_k, a0, k_a [H*head_size]:
 *   u = k k_k, kk = u / max(|u|_row, 1e-12), gate = sigmoid(a0 + a12),
 *   new_k = k (gate k_a + 1 - k_a), neg_kk = -kk, kka = kk gate.
 * io_dtype F16 or BF16 (the reference op is float16 only); head_size 64,
 * 128 or 256; every buffer 16-byte aligned.
 * Replaces tmix_kk_a_gate_forward_varlen
 * (csrc/sm120/tmix/kk_a_gate/infer_fp16_forward_varlen.cu:52-160 and its .cpp).
 */
int frwkv_kk_a_gate(int io_dtype, int64_t total_tokens, int32_t num_heads,
                    int32_t head_size, const void* k, const void* k_k, const void* a0,
                    const void* a12, const void* k_a, void* new_k, void* neg_kk, void* kka,
                    void* stream);

/*
 * TMix consumer of the WKV7 output x, per (token, head) row of packed
 * x, r, k, v, g [total_tokens, H*head_size] with per-channel r_k, weight,
 * bias [H*head_size]:
 *   out = ((x - mean) / sqrt(var + 64e-5) weight + bias + rkv v) g,
 * mean and biased var over the row, rkv = sum_d r k r_k.
 * io_dtype F16 or BF16 (the reference op is float16 only); head_size 64,
 * 128 or 256; every buffer 16-byte aligned.
 * Replaces tmix_lnx_rkvres_xg_forward_varlen
 * (csrc/sm120/tmix/lnx_rkvres_xg/infer_fp16_forward_varlen.cu:56-200 and its .cpp).
 */
int frwkv_lnx_rkvres_xg(int io_dtype, int64_t total_tokens, int32_t num_heads,
                        int32_t head_size, const void* x, const void* r, const void* k,
                        const void* v, const void* r_k, const void* weight, const void* bias,
                        const void* g, void* output, void* stream);

/*
 * Training form of the consumer (the reference's clampw-v3 pretraining
 * pipeline), forward: out as frwkv_lnx_rkvres_xg over tokens [total_tokens,
 * H*head_size] (dense [B,T,C] is total_tokens = B*T) with residual_scale =
 * r_k [H,head_size], and the row statistics mean[total_tokens*H] and
 * rstd[total_tokens*H] (fp32, row = token*H + head, i.e. the reference's
 * [B,T,H]) that the backward reads. io_dtype F16 or BF16 (the reference op is
 * bfloat16 only); token and parameter buffers 16-byte aligned.
 * Replaces pretrain_tmix_lnx_rkvres_xg_cuda
 * (csrc/sm90/tmix/lnx_rkvres_xg/pretrain_bf16_forward.cu:63-126, 318-362;
 * binding pretrain_bf16_forward.cpp:75-98).
 */
int frwkv_lnx_pretrain_forward(int io_dtype, int64_t total_tokens, int32_t num_heads,
                               int32_t head_size, const void* x, const void* r,
                               const void* k, const void* v, const void* residual_scale,
                               const void* weight, const void* bias, const void* g,
                               void* output, float* mean, float* rstd, void* stream);

/* Workspace bytes of frwkv_lnx_pretrain_backward: 3 x H*head_size fp32 per
 * block of 64 tokens. */
size_t frwkv_lnx_pretrain_backward_workspace_bytes(int64_t total_tokens, int32_t num_heads,
                                                   int32_t head_size);

/*
 * Training backward of the consumer: from grad_output and the forward's
 * inputs and row statistics, writes grad_x, grad_r, grad_k, grad_v, grad_g
 * (shaped like x) and grad_residual_scale [H,head_size], grad_weight,
 * grad_bias [H*head_size] (io dtype). The three parameter gradients are sums
 * over all rows, formed per 64-token block in the workspace
 * (frwkv_lnx_pretrain_backward_workspace_bytes, 16-byte aligned) and then
 * added over the blocks in a fixed order, so results are bitwise
 * deterministic. Replaces pretrain_tmix_lnx_rkvres_xg_backward_cuda
 * (csrc/sm90/tmix/lnx_rkvres_xg/pretrain_bf16_backward.cu:125-275, 330-414;
 * binding pretrain_bf16_backward.cpp:83-110).
 */
int frwkv_lnx_pretrain_backward(int io_dtype, int64_t total_tokens, int32_t num_heads,
                                int32_t head_size, const void* grad_output, const void* x,
                                const void* r, const void* k, const void* v,
                                const void* residual_scale, const void* weight,
                                const void* bias, const void* g, const float* mean,
                                const float* rstd, void* grad_x, void* grad_r, void* grad_k,
                                void* grad_v, void* grad_residual_scale, void* grad_weight,
                                void* grad_bias, void* grad_g, void* workspace,
                                size_t workspace_bytes, void* stream);

/*
 * The TMix chain kk_a_gate -> WKV7 recurrent step -> lnx_rkvres_xg in one
 * kernel, for decode and short sequences (fp32 state pool, head_size 64),
 * with no intermediate written to memory and none rounded to 16 bits:
 * the producer gives k' = new_k, a = -kk, b = kk gate (the RWKV-7 update
 * S = diag(w) S + b (a^T S) + k' v^T); y = scale S^T r feeds the consumer
 * with r, k', v. Token tensors r, decay, k, v, a12, g are [total_tokens,H,64]
 * (io dtype), vectors k_k, a0, k_a, r_k, ln_weight, ln_bias [H*64]; output
 * [total_tokens,H,64] is the consumer's result. Metadata, pool and
 * fail-closed behaviour as frwkv_recurrent_forward.
 * No counterpart in the reference, which runs the three stages as separate
 * ops (composed in tests/tmix/wkv7/test.py:310-414); for decode callers that
 * want the producer's three and the consumer's five [N,C] tensors off HBM.
 */
int frwkv_recurrent_tmix_fused_forward(
    int io_dtype, int decay_mode, int32_t num_sequences, int32_t num_heads,
    int32_t head_size, int32_t total_tokens, int32_t state_pool_size,
    const int32_t* cu_seqlens, const int32_t* state_indices, const int32_t* metadata_status,
    float* state_pool, const void* r, const void* decay, const void* decay_bias,
    const void* k, const void* v, const void* a12, const void* g, const void* k_k,
    const void* a0, const void* k_a, const void* r_k, const void* ln_weight,
    const void* ln_bias, void* output, float scale, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FLASHRWKV_AMD_H_ */

// Parameters and chunk walking shared by the head-size-128/256 training
// kernels: the per-token kernels (train_recurrent.hip) and the head-size-128
// MFMA kernels over 16-token pieces (piece_train.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace frwkv {

constexpr int kPiece = 16;  // tokens per piece; the interior checkpoint spacing

// s_waitcnt vmcnt(0), expcnt and lgkmcnt left at their maxima. A state
// loaded before a kernel's piece loop is waited for with it before the loop:
// otherwise the compiler keeps a wait for that load (counting every store in
// flight too) in front of each state store inside the loop.
constexpr int kWaitVmcnt0 = 0x0f70;

struct TrainParams {
  int32_t num_heads;
  int32_t total_tokens;
  int32_t num_sequences;
  // Segmented chunks (StateTune): chunk c of sequence s, c in
  // [seg_offsets[s], seg_offsets[s+1]), covers tokens seg_starts[c] ..
  // seg_ends[c]-1; its start state is ckpt[c, h].
  const int32_t* seg_offsets;
  const int32_t* seg_starts;
  const int32_t* seg_ends;
  int32_t num_chunks;  // length of seg_starts / seg_ends
  // Dense (pretraining): > 0 means sequence s holds tokens s*T .. s*T+T-1 in
  // chunks of 16; chunk j's start state is ckpt[s, h, j] ([B,H,T/16,D,D]).
  int32_t dense_t;
  float* state;        // [B,H,D,D] S0 in, S_T out (forward); null: zero start, no S_T
  float* ckpt;         // chunk start states
  float* state_dot_a;  // [N,H,D] a^T S_{t-1} (forward output)
  const void* r;
  const void* decay;
  const void* bias;    // [H*D] or null (logits mode only)
  const void* k;
  const void* v;
  const void* a;
  const void* b;
  void* out;           // y (forward)
  const void* dy;             // or null (zero)
  const float* dstate_final;  // or null (zero)
  void* dr;
  void* ddecay;
  void* dk;
  void* dv;
  void* da;
  void* db;
  float* dstate0;  // or null
  float* accum;    // [groups, 5, N*H*D] fp32 slices (dr, dk, db, ddecay, da), groups > 1
  float scale;
  // [ceil(N/16), H, D, D] or null: the state at every 16-token piece start
  // inside a chunk (not at the chunk start), at slot (piece start) / 16;
  // interior starts of different chunks lie more than 16 tokens apart, so the
  // slots are distinct. Written by the forward, read by the backward. fp32 at
  // head size 256; bf16 in the piece kernels' lane order at 128.
  float* interior;
  // Forward only: 1 = one chunk per unit (seg_offsets null; chunk c starts from
  // state[c]), only the interior states are written; chunks of at most 16
  // tokens are skipped and a chunk's last piece is not computed.
  int32_t fill_only;
};

struct Chunk {
  int32_t start, end;
  int64_t ckpt_off;  // element offset of the chunk start state
};

// Chunk metadata is read-only for a whole launch: read it through the
// constant address space, so that its (uniform) reads are scalar loads,
// which do not wait for the vector memory operations in flight.
__device__ __forceinline__ int32_t meta_at(const int32_t* a, int i) {
  return ((const __attribute__((address_space(4))) int32_t*)a)[i];
}

__device__ __forceinline__ void chunk_range(const TrainParams& p, int seq, int& c_begin,
                                            int& c_end) {
  if (p.dense_t > 0) {
    c_begin = 0;
    c_end = p.dense_t / kPiece;
  } else if (p.seg_offsets == nullptr) {
    c_begin = seq;
    c_end = min(seq + 1, p.num_chunks);
  } else {
    // Clamped to the chunk arrays, so malformed offsets cannot address
    // outside them.
    c_begin = __builtin_amdgcn_readfirstlane(max(meta_at(p.seg_offsets, seq), 0));
    c_end = __builtin_amdgcn_readfirstlane(min(meta_at(p.seg_offsets, seq + 1), p.num_chunks));
  }
}

template <int D>
__device__ __forceinline__ Chunk chunk_at(const TrainParams& p, int seq, int head, int c) {
  Chunk ch;
  if (p.dense_t > 0) {
    ch.start = seq * p.dense_t + kPiece * c;
    ch.end = ch.start + kPiece;
    ch.ckpt_off = ((static_cast<int64_t>(seq) * p.num_heads + head) * (p.dense_t / kPiece) + c) *
                  static_cast<int64_t>(D) * D;
  } else {
    // Clamped to the token range (an end before the start makes the chunk
    // empty), as the head-size-64 kernels clamp their segments.
    const int32_t start = __builtin_amdgcn_readfirstlane(meta_at(p.seg_starts, c));
    const int32_t end = __builtin_amdgcn_readfirstlane(meta_at(p.seg_ends, c));
    ch.start = min(max(start, 0), p.total_tokens);
    ch.end = max(min(end, p.total_tokens), ch.start);
    ch.ckpt_off = (static_cast<int64_t>(c) * p.num_heads + head) * static_cast<int64_t>(D) * D;
  }
  return ch;
}

// The head-size-128 training forward or backward on bf16 MFMA over 16-token
// pieces (piece_train.hip). Same parameters, outputs and chunk-start states as
// the per-token kernels (one workgroup per unit); interior states in bf16.
int launch_piece_train(const TrainParams& p, int io_dtype, int decay_mode, int units,
                       bool backward, hipStream_t stream);

}  // namespace frwkv

// Multi-row forward in one launch (rows_kernel.h): forward_cached over a
// short prompt of one sequence, or one new token of each of several
// sequences, for f32 weights.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "decode_persistent.h"

namespace rtg {

struct RowsPlan;
// Model geometry check and the per-layer pointer table; null when the model
// is not supported (weights not f32, n_embd not in {128, 768, 1024}, head_dim
// not 64, fewer than 256 CUs).
RowsPlan* rows_plan_create(const PersistentWeights& w, int cus);
void rows_plan_destroy(RowsPlan* p);
// Rows a launch may hold: S sequences x T tokens.
bool rows_supported(const RowsPlan* p, int S, int T);
// Bytes of the state one stream's launches use (flags, epoch, partials and
// activation rows): with fresh, one region per (layer, phase) for the data
// many workgroups read (read with plain loads; ~25 MB for GPT-2 small),
// else one region each (read with device-scope loads, slower; ~2 MB).
size_t rows_state_bytes(const RowsPlan* p, bool fresh);

struct RowsState {
  void* mem = nullptr;  // rows_state_bytes(fresh); the flag words and epoch at its start
  bool owned = false;
  bool fresh = false;
};
// Allocates and initialises a state with layered regions (hipMalloc, zeroed
// flags, epoch 1).
RowsState* rows_state_create(const RowsPlan* p);
// A state may also sit in caller memory of rows_state_bytes (mem set, not
// owned, fresh as sized): its first rows_state_head_bytes (flag words,
// counters, epoch) must hold what the previous launch on that memory left, or
// zeros before the first.
constexpr size_t rows_state_head_bytes() { return 64 * 1024; }
void rows_state_destroy(RowsState* s);
unsigned* rows_err(RowsState* s);

// Enqueues forward_cached of S sequences x T new tokens: ids_dev [S*T], cache
// layer 0 at kc / vc ([seq][head][P][64], kv_layer floats per layer), every
// sequence's first new token at position past, or *pos_dev when pos_dev is
// set; logits [S*T][V]. The caller must hold persistent_launch_lock(device)
// from the launch until the stream has drained.
// With fin set, the launch also finishes a greedy step the way launch_argmax
// + launch_finalize do: keys [S] (zero on entry, cleared again), the argmax
// token of each sequence's last row into token [S] and ids_out[s * ld_ids +
// *step], then *pos and *step advanced by one; for S <= 4 it then computes
// only those last rows' logits (the other rows of logits are not written).
struct RowsFinish {
  unsigned long long* keys;
  uint32_t* token;
  uint32_t* ids_out;
  int ld_ids;
  int* pos;
  int* step;
};
hipError_t rows_forward(const RowsPlan* p, RowsState* s, hipStream_t stream, float* kc, float* vc, long kv_layer,
                        const uint32_t* ids_dev, int S, int T, int past, const int* pos_dev, float* logits,
                        const RowsFinish* fin = nullptr, uint64_t* trace = nullptr);
// With $RTG_ROWS_TRACE set, every launch records per-workgroup phase
// timestamps (100 MHz clock; [256][512] u64: word 2 (8 (l + 1) + phase) + k,
// k = 0 inputs ready, 1 outputs published; the LM head is layer L, phase 0;
// the last word the workgroup's start) and this writes the latest launch's to
// that file, after the caller has drained the stream.
void rows_dump_trace();

}  // namespace rtg

// kvcache_internal.h -- the KV-cache handle's stream-ordered pieces, shared by
// the C ABI (api.hip, which owns the handle) and the resident MHA (mha.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

#include <vector>

#include "../../include/gonn_hip.h"

namespace gonn {

// Batch, heads, capacity and head dim of a cache handle.
void kvcache_dims(const gonn_kvcache* c, int* B, int* H, int* Lmax, int* D);
// Enqueues on s the append of T rows of every sequence (k, v: f32 device
// (B,H,T,D)) and the upload of the new lengths to the device copy; the new
// lengths go to *new_len. Nothing is committed: the caller synchronises s and
// then calls kvcache_commit, or kvcache_restore after a failure.
int kvcache_append_pending(gonn_kvcache* c, const float* k, const float* v, int T, hipStream_t s,
                           std::vector<int>* new_len);
void kvcache_commit(gonn_kvcache* c, std::vector<int>* new_len);
// Puts the committed lengths back on the device (after a failed call). If
// that copy fails too, the handle is marked stale: every later call that
// reads the device lengths returns GONN_E_INVALID until a successful
// gonn_hip_kvcache_reset. Returns the copy's status.
int kvcache_restore(gonn_kvcache* c);
// False for a stale handle (see kvcache_restore).
bool kvcache_usable(const gonn_kvcache* c);
// Workspace of the causal multi-token attend of T queries per (b,h).
size_t kvcache_attend_causal_ws(const gonn_kvcache* c, int T);
// Enqueues the causal multi-token attend: q, o f32 device (B,H,T,D); query t
// sees cached keys [0, len_b - (T - 1 - t)) with the lengths of the device
// copy at that point of the stream.
int kvcache_attend_causal_run(gonn_kvcache* c, const float* q, float* o, int T, double scale,
                              void* ws, hipStream_t s, bool profile);

}  // namespace gonn

// Work distribution of the ping-pong attention kernels: the XCD-aware deal of
// work items to workgroups, and the per-XCD work queues of the persistent
// grid.  Host and device code, so that the arithmetic and the take-with-
// stealing order can be checked exhaustively on the CPU.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

namespace h3a {

// Dispatch index i of a grid whose workgroups the hardware deals round-robin
// over 8 XCDs -> work item, so that each XCD walks one contiguous range of
// work items (consecutive query tiles of the same head), which keeps that
// head's K/V stream resident in the XCD's own L2.  Bijective for any total.
__host__ __device__ __forceinline__ int xcd_remap(int i, int total) {
  constexpr int kXcds = 8;
  const int per = total / kXcds, rem = total % kXcds;
  const int x = i % kXcds, idx = i / kXcds;
  return x * per + (x < rem ? x : rem) + idx;
}

// Dynamic dispatch: kQueues queues, one per XCD.  Queue x holds XCD x's share
// of the whole work items (the contiguous range xcd_remap deals it) followed by
// its share of the split pieces.  A workgroup takes items from its own XCD's
// queue and, once that is empty, from the others in turn, so XCDs that run at
// a higher clock finish the slower ones' work instead of idling.  Each queue
// is a counter in its own 128-byte line (kQueueStride ints), zeroed before
// every launch.
constexpr int kQueues = 8;
constexpr int kQueueStride = 32;
constexpr size_t kSchedBytes = (size_t)kQueues * kQueueStride * sizeof(int);

struct QueueShare {
  int first, len;
};
__host__ __device__ __forceinline__ QueueShare queue_share(int n, int x) {
  const int per = n / kQueues, rem = n % kQueues;
  return {x * per + (x < rem ? x : rem), per + (x < rem ? 1 : 0)};
}

// Items in queue x, and the work item at position i < queue_len of it (items
// 0..whole-1 are whole tiles, whole + p is split piece p).
__host__ __device__ __forceinline__ int queue_len(int whole, int pieces, int x) {
  return queue_share(whole, x).len + queue_share(pieces, x).len;
}
__host__ __device__ __forceinline__ int queue_item(int whole, int pieces, int x, int i) {
  const QueueShare sw = queue_share(whole, x), sp = queue_share(pieces, x);
  return i < sw.len ? sw.first + i : whole + sp.first + (i - sw.len);
}

// The next work item for a workgroup on XCD xcc (0 <= xcc < kQueues), or -1
// when every queue is empty: its own queue first, then the others in turn.  load(x) reads queue
// x's counter, fetch_add(x) increments it and returns the old value (agent-
// scope atomics on the GPU).  A counter may run past its queue's length; such
// takes find nothing.  A take can be split in two: the fetch-add on the own
// queue first (its value, `own`, is only needed later), then take_finish.
template <class Load, class FetchAdd>
__host__ __device__ __forceinline__ int take_finish(int whole, int pieces, int xcc, int own, Load load,
                                                    FetchAdd fetch_add) {
  if (own < queue_len(whole, pieces, xcc)) return queue_item(whole, pieces, xcc, own);
  for (int t = 1; t < kQueues; ++t) {
    const int x = (xcc + t) & (kQueues - 1);
    const int len = queue_len(whole, pieces, x);
    if (load(x) >= len) continue;
    const int i = fetch_add(x);
    if (i < len) return queue_item(whole, pieces, x, i);
  }
  return -1;
}

template <class Load, class FetchAdd>
__host__ __device__ __forceinline__ int take_item_with(int whole, int pieces, int xcc, Load load,
                                                       FetchAdd fetch_add) {
  return take_finish(whole, pieces, xcc, fetch_add(xcc), load, fetch_add);
}

}  // namespace h3a

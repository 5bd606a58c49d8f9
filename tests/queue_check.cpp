// Exhaustive check of the ping-pong kernels' work distribution
// (minimaxh3-on-a100-x4_amd/csrc/h3a_queue.h) on the host: the XCD-aware deal
// xcd_remap, the per-XCD queue shares, and the take-with-stealing order under
// concurrent workgroups (threads over std::atomic counters).
// Built and run by tests/test_queue_arith.py; prints "OK" or the first failure.
#include <atomic>
#include <cstdio>
#include <random>
#include <thread>
#include <vector>

#include "h3a_queue.h"

using h3a::kQueues;

#define CHECK(c, ...)              \
  do {                             \
    if (!(c)) {                    \
      printf(__VA_ARGS__);         \
      printf("\n");                \
      return false;                \
    }                              \
  } while (0)

// Shares of n items over the queues: in queue order, contiguous, disjoint,
// covering [0, n), lengths differing by at most one; and queue x's share is
// exactly the set of work items xcd_remap deals the dispatch indices of XCD x
// (i % 8 == x), which must be a bijection of [0, n).
static bool check_shares(int n) {
  int next = 0, lo = n, hi = 0;
  for (int x = 0; x < kQueues; ++x) {
    const h3a::QueueShare s = h3a::queue_share(n, x);
    CHECK(s.first == next && s.len >= 0, "n=%d x=%d: share (%d,%d) does not start at %d", n, x, s.first, s.len, next);
    next += s.len;
    lo = s.len < lo ? s.len : lo;
    hi = s.len > hi ? s.len : hi;
  }
  CHECK(next == n, "n=%d: shares cover %d items", n, next);
  CHECK(hi - lo <= 1, "n=%d: share lengths %d..%d", n, lo, hi);
  std::vector<int> seen(n, 0);
  for (int i = 0; i < n; ++i) {
    const int w = h3a::xcd_remap(i, n);
    CHECK(w >= 0 && w < n, "n=%d: xcd_remap(%d) = %d out of range", n, i, w);
    CHECK(!seen[w]++, "n=%d: xcd_remap hits item %d twice", n, w);
    const h3a::QueueShare s = h3a::queue_share(n, i % kQueues);
    CHECK(w >= s.first && w < s.first + s.len, "n=%d: dispatch %d (XCD %d) -> item %d outside queue share [%d,%d)",
          n, i, i % kQueues, w, s.first, s.first + s.len);
  }
  return true;
}

// queue_item over every (queue, position) lists each of the whole + pieces
// work items exactly once, whole tiles first within each queue.
static bool check_items(int whole, int pieces) {
  std::vector<int> seen(whole + pieces, 0);
  int total = 0;
  for (int x = 0; x < kQueues; ++x) {
    const int len = h3a::queue_len(whole, pieces, x);
    total += len;
    bool in_pieces = false;
    for (int i = 0; i < len; ++i) {
      const int it = h3a::queue_item(whole, pieces, x, i);
      CHECK(it >= 0 && it < whole + pieces, "whole=%d pieces=%d: queue %d pos %d -> %d", whole, pieces, x, i, it);
      CHECK(!seen[it]++, "whole=%d pieces=%d: item %d in two places", whole, pieces, it);
      CHECK(!(in_pieces && it < whole), "whole=%d pieces=%d: queue %d has a whole tile after a piece", whole, pieces, x);
      in_pieces = it >= whole;
    }
  }
  CHECK(total == whole + pieces, "whole=%d pieces=%d: queues hold %d items", whole, pieces, total);
  return true;
}

// Sequential takes, one workgroup per XCD taking in turn: each take returns
// the next item of the taker's own queue while that queue has one, else the
// next item of the first non-empty queue after it (in queue order, wrapping).
static bool check_order(int whole, int pieces) {
  std::vector<int> ctr(kQueues, 0);
  auto load = [&](int q) { return ctr[q]; };
  auto add = [&](int q) { return ctr[q]++; };
  int handed = 0;
  for (int round = 0; handed < whole + pieces; ++round) {
    CHECK(round <= whole + pieces, "whole=%d pieces=%d: takes do not end", whole, pieces);
    for (int xcc = 0; xcc < kQueues; ++xcc) {
      int want = -1;
      for (int t = 0; t < kQueues && want < 0; ++t) {
        const int x = (xcc + t) % kQueues;
        if (ctr[x] < h3a::queue_len(whole, pieces, x)) want = h3a::queue_item(whole, pieces, x, ctr[x]);
      }
      const int it = h3a::take_item_with(whole, pieces, xcc, load, add);
      CHECK(it == want, "whole=%d pieces=%d: XCD %d took item %d, want %d", whole, pieces, xcc, it, want);
      handed += it >= 0;
    }
  }
  for (int xcc = 0; xcc < kQueues; ++xcc)
    CHECK(h3a::take_item_with(whole, pieces, xcc, load, add) == -1, "whole=%d pieces=%d: take after the end", whole,
          pieces);
  return true;
}

// Workgroups as threads taking concurrently through std::atomic counters
// (relaxed, as on the GPU), each until it gets -1, as the kernel's item loop
// does, half of the takes split into the own queue's fetch-add and a later
// take_finish.  Checks: every item handed out exactly once, and once any take
// returns -1 every queue's counter has reached its length (all items claimed).
static bool check_concurrent(int whole, int pieces, int threads, unsigned seed) {
  const int n = whole + pieces;
  std::vector<std::atomic<int>> ctr(kQueues);
  for (auto &c : ctr) c.store(0);
  std::vector<std::atomic<int>> seen(n > 0 ? n : 1);
  for (auto &s : seen) s.store(0);
  std::atomic<int> bad{0};
  std::vector<std::thread> pool;
  for (int w = 0; w < threads; ++w)
    pool.emplace_back([&, w] {
      std::mt19937 rng(seed * 1000003u + (unsigned)w);
      const int xcc = (int)(rng() % kQueues);
      auto load = [&](int q) { return ctr[q].load(std::memory_order_relaxed); };
      auto add = [&](int q) { return ctr[q].fetch_add(1, std::memory_order_relaxed); };
      for (;;) {
        if (rng() % 4 == 0) std::this_thread::yield();
        int it;
        if (rng() % 2) {
          it = h3a::take_item_with(whole, pieces, xcc, load, add);
        } else {
          // The split take: the own queue's fetch-add, other takers, then the
          // finish (as a work item's epilogue runs between the two halves).
          const int own = add(xcc);
          std::this_thread::yield();
          it = h3a::take_finish(whole, pieces, xcc, own, load, add);
        }
        if (it < 0) {
          for (int q = 0; q < kQueues; ++q)
            if (ctr[q].load() < h3a::queue_len(whole, pieces, q)) bad.fetch_or(1);
          return;
        }
        if (it >= n) {
          bad.fetch_or(2);
          return;
        }
        seen[it].fetch_add(1);
      }
    });
  for (auto &t : pool) t.join();
  CHECK(!(bad.load() & 1), "whole=%d pieces=%d threads=%d: -1 while items were unclaimed", whole, pieces, threads);
  CHECK(!(bad.load() & 2), "whole=%d pieces=%d threads=%d: item out of range", whole, pieces, threads);
  for (int i = 0; i < n; ++i)
    CHECK(seen[i].load() == 1, "whole=%d pieces=%d threads=%d: item %d handed out %d times", whole, pieces, threads, i,
          seen[i].load());
  return true;
}

int main() {
  for (int n = 0; n <= 5000; ++n)
    if (!check_shares(n)) return 1;
  for (int n : {9240, 18480, 36960, 73920, 1 << 20, (1 << 20) + 7})
    if (!check_shares(n)) return 1;
  for (int whole = 0; whole <= 260; ++whole)
    for (int pieces = 0; pieces <= 40; ++pieces)
      if (!check_items(whole, pieces) || !check_order(whole, pieces)) return 1;
  // The bench shapes: 9,240 128-row pairs / 18,480 64-row pairs of the
  // sparse path (H=56, S=42120), 18,480 dense tiles, and ragged ones.
  for (int whole : {9240, 18480, 4105, 2049})
    for (int pieces : {0, 7, 256})
      if (!check_items(whole, pieces) || !check_order(whole, pieces)) return 1;
  unsigned seed = 1;
  for (int whole : {0, 1, 7, 8, 9, 255, 256, 1000, 9240})
    for (int pieces : {0, 1, 13, 512})
      for (int threads : {1, 8, 33})
        if (!check_concurrent(whole, pieces, threads, seed++)) return 1;
  printf("OK\n");
  return 0;
}

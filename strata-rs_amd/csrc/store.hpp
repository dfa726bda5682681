// Eviction policy of the resident weight store (host code, no device calls).
//
// The store is the reference GPU backend's weight cache
// (crates/strata-backend-wgpu/src/gpu.rs:61-113): entries keyed by tensor,
// bounded by a byte budget, least-recently-used evicted first until a new
// entry fits, and a single entry larger than the budget still admitted alone.
//
// One difference: an entry point here may need several tensors at once (the
// MoE and FFN calls hold up to eight), and admitting a later tensor must not
// evict an earlier one of the same call, whose device pointer the call is
// about to launch on. Every admission therefore stamps its entry with the
// current call number (`pin`), and entries stamped by the current call are
// never victims. When the unpinned entries cannot make room, the admission
// fails (the caller reports out-of-memory before any launch).
#pragma once

#include <stdint.h>

#include <algorithm>
#include <vector>

namespace sh {

struct StoreEntry {
  uint64_t key;
  uint64_t bytes;
  uint64_t used;  // LRU clock of the last admission or hit
  uint64_t pin;   // call number of the last admission or hit
};

// Chooses the entries to evict so that `incoming` more bytes fit beside
// `total` resident bytes under `budget`, least recently used first, skipping
// entries pinned by call `call`. Fills `victims` (keys, in eviction order)
// and returns true when the new entry can be admitted: either it fits, or
// every resident entry is evicted (the store then holds the new entry alone,
// as gpu.rs:88-112 admits a tensor larger than the budget). Returns false,
// with `victims` empty, when entries pinned by `call` stay and the budget
// cannot hold them and the new entry together.
inline bool plan_eviction(const std::vector<StoreEntry>& entries, uint64_t total, uint64_t budget,
                          uint64_t incoming, uint64_t call, std::vector<uint64_t>* victims) {
  victims->clear();
  if (total + incoming <= budget && total + incoming >= total) return true;
  std::vector<const StoreEntry*> order;
  order.reserve(entries.size());
  bool pinned = false;
  for (const StoreEntry& e : entries) {
    if (e.pin == call) pinned = true;
    else order.push_back(&e);
  }
  std::sort(order.begin(), order.end(), [](const StoreEntry* a, const StoreEntry* b) {
    return a->used != b->used ? a->used < b->used : a->key < b->key;
  });
  uint64_t left = total;
  for (const StoreEntry* e : order) {
    if (left + incoming <= budget && left + incoming >= left) break;
    victims->push_back(e->key);
    left -= e->bytes;
  }
  const bool fits = left + incoming <= budget && left + incoming >= left;
  if (fits || !pinned) return true;  // an empty store admits anything, alone
  victims->clear();
  return false;
}

}  // namespace sh

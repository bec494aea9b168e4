// Device prefix store: the engine's PrefixCache (crates/cev-model/src/engine.rs:474-503)
// over slot ranges of per-layer device K/V caches, host bookkeeping only.
//
// The reference keeps every cached prefix as its own refcounted K/V tensors
// and concatenates the pasts of a pass's plans (engine.rs:367-387) and a
// plan's head with its freshly computed tail (engine.rs:445-461).  Here
// every layer owns one (hkv, capacity, d) cache, the same slot numbering in
// each layer, and a prefix is a contiguous slot range in it:
//   - a miss reserves the whole prefix's range up front; the prefill writes
//     the head and the packed pass the tail in place, so the extended prefix
//     is already contiguous (no cat);
//   - the attention table points each plan's blocks at that plan's range,
//     so several plans' pasts are read where they lie (no concatenation);
//   - question tokens get a scratch range for the pass.
// LRU semantics are PrefixCache's: get() moves a hit to the back, put()
// replaces an entry with the same key, appends, and evicts from the front
// while the entries' key lengths sum above the budget; a key longer than the
// budget is not cached.  A range stays allocated while a pass holds it
// (pinned, as a plan's Arc keeps the reference's K/V alive), also after
// eviction.  One difference: when no free run of slots fits a reservation,
// the oldest unpinned entries are evicted until one does (fragmentation;
// with capacity >= budget + the largest pass's working set that only
// happens when free slots are scattered), and CEV_ERR_SPACE is returned if
// none fits even then.
#include <stdint.h>

#include <algorithm>
#include <iterator>
#include <map>
#include <mutex>
#include <vector>

#include "cev_internal.h"

namespace {

struct Range {
  int32_t len;
  int32_t pins;   // passes holding the range
  bool entry;     // owned by a cache entry
};

struct Entry {
  std::vector<uint32_t> key;
  int32_t begin;
};

struct Store {
  int32_t capacity;
  int64_t budget;
  std::mutex mu;
  std::map<int32_t, Range> ranges;  // allocated ranges by first slot
  std::vector<Entry> entries;       // LRU order: front = oldest

  int64_t cached_tokens() const {
    int64_t n = 0;
    for (const Entry& e : entries) n += (int64_t)e.key.size();
    return n;
  }

  void maybe_free(std::map<int32_t, Range>::iterator it) {
    if (it->second.pins == 0 && !it->second.entry) ranges.erase(it);
  }

  // Drops entry i; its range is freed unless a pass still holds it.
  void drop_entry(size_t i) {
    auto it = ranges.find(entries[i].begin);
    entries.erase(entries.begin() + (std::ptrdiff_t)i);
    if (it != ranges.end()) {
      it->second.entry = false;
      maybe_free(it);
    }
  }

  // First free run of n slots, or -1.
  int32_t first_fit(int32_t n) const {
    int32_t pos = 0;
    for (const auto& kv : ranges) {
      if (kv.first - pos >= n) return pos;
      pos = std::max(pos, kv.first + kv.second.len);
    }
    return capacity - pos >= n ? pos : -1;
  }
};

Store* as_store(cev_prefix_store s) { return (Store*)s; }

}  // namespace

extern "C" int32_t cev_prefix_store_create(int32_t capacity, int64_t budget, cev_prefix_store* out) {
  CEV_CHECK_ARG(out != nullptr, "cev_prefix_store_create: null output");
  CEV_CHECK_ARG(capacity > 0 && budget >= 0, "cev_prefix_store_create: capacity %d, budget %lld", capacity, (long long)budget);
  Store* s = new Store;
  s->capacity = capacity;
  s->budget = budget;
  *out = s;
  return CEV_OK;
}

extern "C" int32_t cev_prefix_store_destroy(cev_prefix_store store) {
  delete as_store(store);
  return CEV_OK;
}

extern "C" int32_t cev_prefix_store_get(cev_prefix_store store, const uint32_t* tokens, int32_t n, int32_t* begin, int32_t* found) {
  Store* s = as_store(store);
  CEV_CHECK_ARG(s && begin && found && n >= 0 && (n == 0 || tokens), "cev_prefix_store_get: bad arguments");
  std::lock_guard<std::mutex> lock(s->mu);
  *found = 0;
  *begin = -1;
  for (size_t i = 0; i < s->entries.size(); ++i) {
    const Entry& e = s->entries[i];
    if ((int32_t)e.key.size() != n || !std::equal(e.key.begin(), e.key.end(), tokens)) continue;
    Entry hit = e;
    s->entries.erase(s->entries.begin() + (std::ptrdiff_t)i);
    s->entries.push_back(hit);
    s->ranges[hit.begin].pins++;
    *begin = hit.begin;
    *found = 1;
    return CEV_OK;
  }
  return CEV_OK;
}

extern "C" int32_t cev_prefix_store_reserve(cev_prefix_store store, int32_t n, int32_t* begin) {
  Store* s = as_store(store);
  CEV_CHECK_ARG(s && begin && n >= 1, "cev_prefix_store_reserve: bad arguments");
  std::lock_guard<std::mutex> lock(s->mu);
  int32_t at = s->first_fit(n);
  while (at < 0) {
    auto it = std::find_if(s->entries.begin(), s->entries.end(), [&](const Entry& e) { return s->ranges[e.begin].pins == 0; });
    if (it == s->entries.end()) break;
    s->drop_entry((size_t)std::distance(s->entries.begin(), it));
    at = s->first_fit(n);
  }
  if (at < 0) return cev_fail(CEV_ERR_SPACE, "cev_prefix_store_reserve: no run of %d free slots in %d (every range is held)", n, s->capacity);
  s->ranges[at] = Range{n, 1, false};
  *begin = at;
  return CEV_OK;
}

extern "C" int32_t cev_prefix_store_put(cev_prefix_store store, const uint32_t* tokens, int32_t n, int32_t begin) {
  Store* s = as_store(store);
  CEV_CHECK_ARG(s && n >= 1 && tokens, "cev_prefix_store_put: bad arguments");
  std::lock_guard<std::mutex> lock(s->mu);
  auto it = s->ranges.find(begin);
  CEV_CHECK_ARG(it != s->ranges.end() && !it->second.entry && it->second.pins > 0 && it->second.len == n,
                "cev_prefix_store_put: slots [%d, %d) are not a held reservation of %d slots", begin, begin + n, n);
  if ((int64_t)n > s->budget) return CEV_OK;  // not cached (engine.rs:494-496); the caller still releases it
  for (size_t i = 0; i < s->entries.size(); ++i)
    if ((int32_t)s->entries[i].key.size() == n && std::equal(tokens, tokens + n, s->entries[i].key.begin())) {
      s->drop_entry(i);
      break;
    }
  it = s->ranges.find(begin);
  it->second.entry = true;
  s->entries.push_back(Entry{std::vector<uint32_t>(tokens, tokens + n), begin});
  while (s->cached_tokens() > s->budget) s->drop_entry(0);
  return CEV_OK;
}

extern "C" int32_t cev_prefix_store_release(cev_prefix_store store, int32_t begin) {
  Store* s = as_store(store);
  CEV_CHECK_ARG(s != nullptr, "cev_prefix_store_release: null store");
  std::lock_guard<std::mutex> lock(s->mu);
  auto it = s->ranges.find(begin);
  CEV_CHECK_ARG(it != s->ranges.end() && it->second.pins > 0, "cev_prefix_store_release: slot %d is not held", begin);
  it->second.pins--;
  s->maybe_free(it);
  return CEV_OK;
}

extern "C" int32_t cev_prefix_store_stats(cev_prefix_store store, int32_t* entries, int64_t* cached_tokens, int32_t* used_slots) {
  Store* s = as_store(store);
  CEV_CHECK_ARG(s != nullptr, "cev_prefix_store_stats: null store");
  std::lock_guard<std::mutex> lock(s->mu);
  if (entries) *entries = (int32_t)s->entries.size();
  if (cached_tokens) *cached_tokens = s->cached_tokens();
  if (used_slots) {
    int64_t u = 0;
    for (const auto& kv : s->ranges) u += kv.second.len;
    *used_slots = (int32_t)u;
  }
  return CEV_OK;
}

extern "C" int32_t cev_prefix_store_entry(cev_prefix_store store, int32_t i, int32_t* begin, int32_t* len) {
  Store* s = as_store(store);
  CEV_CHECK_ARG(s && begin && len, "cev_prefix_store_entry: bad arguments");
  std::lock_guard<std::mutex> lock(s->mu);
  CEV_CHECK_ARG(i >= 0 && i < (int32_t)s->entries.size(), "cev_prefix_store_entry: entry %d of %zu", i, s->entries.size());
  *begin = s->entries[(size_t)i].begin;
  *len = (int32_t)s->entries[(size_t)i].key.size();
  return CEV_OK;
}

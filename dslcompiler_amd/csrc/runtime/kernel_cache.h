// kernel_cache.h -- four-level LRU cache of the gfx950 backend, the
// counterpart of the reference's JitCache (include/LLK/Runtime/JitCache.h:
// 67-218, runtime/JitCache.cpp:41-88, 247-397).
//
//   L1  string -> string      (the reference's IR level; opaque text here)
//   L2  string -> string      (the reference's optimized-MLIR level)
//   L3  KernelKey -> entry    (object code: a precompiled gfx950 entry point)
//   L4  WeightKey -> handle   (device-resident packed weights, owned)
//
// Every level keeps the reference's LRU rules: a hit moves the entry to the
// most-recently-used end; inserting a new key first evicts from the least-
// recently-used end while the level holds max_entries (default 1024) or
// more; inserting an existing key replaces its value and refreshes it;
// evict(n) trims to at most n entries and makes n the level's capacity.
// Each level has its own reader/writer lock and hit/miss/eviction counters.
#pragma once

#include <cstddef>
#include <cstdint>
#include <list>
#include <memory>
#include <mutex>
#include <shared_mutex>
#include <string>
#include <unordered_map>
#include <utility>

namespace llk {

template <class V>
class LruLevel {
 public:
  // Copies the value of `key` into *out and refreshes it; false on a miss.
  bool lookup(const std::string& key, V* out) {
    std::unique_lock<std::shared_mutex> lk(mu_);  // splice mutates the list
    auto it = index_.find(key);
    if (it == index_.end()) {
      ++misses_;
      return false;
    }
    ++hits_;
    order_.splice(order_.begin(), order_, it->second);
    if (out) *out = it->second->second;
    return true;
  }

  void insert(const std::string& key, V value) {
    std::unique_lock<std::shared_mutex> lk(mu_);
    auto it = index_.find(key);
    if (it != index_.end()) {
      it->second->second = std::move(value);
      order_.splice(order_.begin(), order_, it->second);
      return;
    }
    while (!order_.empty() && order_.size() >= max_entries_) pop_back();
    order_.emplace_front(key, std::move(value));
    index_[key] = order_.begin();
  }

  // insert() whose value is made only when needed: if `key` holds a value
  // for which same(value) is true, that entry is just refreshed and make()
  // is not called (an owning value for the same object is never made twice).
  // If an allocation throws, the level is left as it was.
  template <class Same, class Make>
  void insert_with(const std::string& key, Same same, Make make) {
    std::unique_lock<std::shared_mutex> lk(mu_);
    auto it = index_.find(key);
    if (it != index_.end()) {
      if (!same(it->second->second)) it->second->second = make();
      order_.splice(order_.begin(), order_, it->second);
      return;
    }
    while (!order_.empty() && order_.size() >= max_entries_) pop_back();
    auto slot = index_.emplace(key, order_.end()).first;
    try {
      order_.emplace_front(key, make());
    } catch (...) {
      index_.erase(slot);
      throw;
    }
    slot->second = order_.begin();
  }

  bool remove(const std::string& key) {
    std::unique_lock<std::shared_mutex> lk(mu_);
    auto it = index_.find(key);
    if (it == index_.end()) return false;
    order_.erase(it->second);
    index_.erase(it);
    return true;
  }

  void evict(size_t max_entries) {
    std::unique_lock<std::shared_mutex> lk(mu_);
    while (!order_.empty() && order_.size() > max_entries) pop_back();
    max_entries_ = max_entries;
  }

  void clear() {
    std::unique_lock<std::shared_mutex> lk(mu_);
    index_.clear();
    order_.clear();
  }

  size_t size() const {
    std::shared_lock<std::shared_mutex> lk(mu_);
    return index_.size();
  }

  void stats(size_t* hits, size_t* misses, size_t* evictions) const {
    std::shared_lock<std::shared_mutex> lk(mu_);
    *hits = hits_;
    *misses = misses_;
    *evictions = evictions_;
  }

 private:
  void pop_back() {
    index_.erase(order_.back().first);
    order_.pop_back();
    ++evictions_;
  }

  std::list<std::pair<std::string, V>> order_;  // front = most recently used
  std::unordered_map<std::string, typename std::list<std::pair<std::string, V>>::iterator> index_;
  size_t max_entries_ = 1024;
  size_t hits_ = 0, misses_ = 0, evictions_ = 0;
  mutable std::shared_mutex mu_;
};

}  // namespace llk

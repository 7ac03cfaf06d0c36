// A process-lifetime map from a key to one object made on the key's first request (host code).
//
// The prefill entry points keep one side stream per (device, caller stream) in such a map: distinct keys get
// distinct objects, a key gets the same object on every later request, and concurrent first requests of one key
// from several threads make it once.  Objects are never destroyed (HIP streams and events may still have work
// queued when the process ends).  Header-only and free of HIP types so a CPU test can exercise it.
#pragma once
#include <map>
#include <memory>
#include <mutex>

namespace mimo {

template <class Key, class T>
class KeyedOnce {
 public:
  // The object of `key`, made by make() (a std::unique_ptr<T>, empty on failure) on the first request; nullptr
  // when making it failed (a later request tries again) or when `cap` objects exist already and `key` has none
  // (the map never holds more than `cap` objects).
  template <class Make>
  T* get(const Key& key, Make make, size_t cap = (size_t)-1) {
    std::lock_guard<std::mutex> g(mu_);
    auto it = map_.find(key);
    if (it != map_.end() && it->second) return it->second.get();
    if (made_ >= cap) return nullptr;
    std::unique_ptr<T> obj = make();
    if (!obj) return nullptr;
    T* ptr = obj.get();
    map_[key] = std::move(obj);
    ++made_;
    return ptr;
  }
  size_t size() {
    std::lock_guard<std::mutex> g(mu_);
    return made_;
  }

 private:
  std::mutex mu_;
  std::map<Key, std::unique_ptr<T>> map_;
  size_t made_ = 0;
};

}  // namespace mimo

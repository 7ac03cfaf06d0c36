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
  // when making it failed (a later request tries again).
  template <class Make>
  T* get(const Key& key, Make make) {
    std::lock_guard<std::mutex> g(mu_);
    std::unique_ptr<T>& slot = map_[key];
    if (!slot) slot = make();
    return slot.get();
  }
  size_t size() {
    std::lock_guard<std::mutex> g(mu_);
    size_t n = 0;
    for (auto& kv : map_) n += kv.second ? 1 : 0;
    return n;
  }

 private:
  std::mutex mu_;
  std::map<Key, std::unique_ptr<T>> map_;
};

}  // namespace mimo

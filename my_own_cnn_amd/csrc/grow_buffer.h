// Grow-only device buffers for the entry points whose signature (the reference's) has no
// workspace argument: the float-code row-band and stream paths keep one per (device, stream),
// the fp32 filter gradient one per device.
//
// A buffer is never freed while the process runs.  When a larger problem arrives, a new
// buffer of at least twice the capacity is allocated and the old one is retired, not freed:
// work already enqueued on a stream, or recorded in a captured graph, may still read it, and
// freeing it safely would need a synchronisation inside an asynchronous call.  Because each
// growth at least doubles the capacity, the retired buffers of one entry together stay
// smaller than its live buffer.  The table of entries has a fixed limit; a new key beyond it
// is refused and the caller reports an error that names the caller-workspace form.
//
// Pure host code with the allocator passed in, so the growth and retirement rules are tested
// on the CPU with a fake allocator.
#ifndef MIQ_GROW_BUFFER_H_
#define MIQ_GROW_BUFFER_H_

#include <algorithm>
#include <cstddef>
#include <deque>
#include <utility>
#include <vector>

namespace miq {

struct GrowBuffer {
  void* p = nullptr;
  size_t bytes = 0;              // capacity of p
  std::vector<void*> retired;    // earlier buffers, kept until the process ends
};

// Makes b hold at least `need` bytes and returns the live buffer in *out.  `alloc(void**,
// size_t)` returns 0 on success; when the doubled capacity cannot be allocated, exactly
// `need` is tried.  On failure b is unchanged and alloc's status is returned.
template <typename Alloc>
int grow_buffer(GrowBuffer& b, size_t need, Alloc&& alloc, void** out) {
  *out = nullptr;
  if (b.bytes < need) {
    const size_t doubled = b.bytes > (static_cast<size_t>(-1) >> 1) ? need : 2 * b.bytes;
    size_t cap = std::max(need, doubled);
    void* np = nullptr;
    int st = alloc(&np, cap);
    if (st != 0 && cap > need) {
      cap = need;
      st = alloc(&np, cap);
    }
    if (st != 0) return st;
    if (b.p != nullptr) b.retired.push_back(b.p);
    b.p = np;
    b.bytes = cap;
  }
  *out = b.p;
  return 0;
}

// At most `limit` keyed GrowBuffers; entries live until the process ends (their addresses
// stay valid: a deque does not move its elements when it grows at the end).  Not locked:
// the caller holds its own mutex around find_or_add and grow_buffer.
template <typename Key>
class GrowBufferTable {
 public:
  explicit GrowBufferTable(size_t limit) : limit_(limit) {}

  // The key's entry, created empty on first use; nullptr when the key is new and the table
  // already holds `limit` entries.
  GrowBuffer* find_or_add(const Key& k) {
    for (auto& e : entries_) {
      if (e.first == k) return &e.second;
    }
    if (entries_.size() >= limit_) return nullptr;
    entries_.emplace_back(k, GrowBuffer{});
    return &entries_.back().second;
  }

  size_t size() const { return entries_.size(); }

 private:
  size_t limit_;
  std::deque<std::pair<Key, GrowBuffer>> entries_;
};

}  // namespace miq

#endif  // MIQ_GROW_BUFFER_H_

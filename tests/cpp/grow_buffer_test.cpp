// Host-only test of the grow-only workspace rules (my_own_cnn_amd/csrc/grow_buffer.h) with a
// fake allocator: growth at least doubles, outgrown buffers are retired and never freed, a
// failed doubled request falls back to the exact size, a failed allocation leaves the entry
// unchanged, and the keyed table keeps its limit and stable entry addresses.  Built and run by
// tests/test_grow_buffer.py with g++ (no GPU).  Prints "ok" and exits 0 on success.
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "grow_buffer.h"

namespace {

int failures = 0;
#define CHECK(cond)                                                        \
  do {                                                                     \
    if (!(cond)) {                                                         \
      std::printf("FAILED line %d: %s\n", __LINE__, #cond);                \
      ++failures;                                                          \
    }                                                                      \
  } while (0)

// Hands out distinct fake addresses; refuses requests above `limit` bytes.
struct FakeAlloc {
  size_t limit = static_cast<size_t>(-1);
  std::vector<size_t> requests;
  char* next = reinterpret_cast<char*>(0x10000);
  int operator()(void** p, size_t bytes) {
    requests.push_back(bytes);
    if (bytes > limit) return 7;
    *p = next;
    next += bytes + 4096;
    return 0;
  }
};

}  // namespace

int main() {
  using miq::GrowBuffer;
  using miq::grow_buffer;
  FakeAlloc fa;
  GrowBuffer b;
  void* out = nullptr;

  CHECK(grow_buffer(b, 100, fa, &out) == 0);
  CHECK(out == b.p && b.bytes == 100 && b.retired.empty() && fa.requests.size() == 1);
  void* first = out;

  CHECK(grow_buffer(b, 50, fa, &out) == 0);  // fits: no allocation
  CHECK(out == first && fa.requests.size() == 1);

  CHECK(grow_buffer(b, 150, fa, &out) == 0);  // doubled: 200
  CHECK(b.bytes == 200 && out != first && b.retired.size() == 1 && b.retired[0] == first);

  CHECK(grow_buffer(b, 1000, fa, &out) == 0);  // need beyond double: exactly 1000
  CHECK(b.bytes == 1000 && b.retired.size() == 2);
  CHECK(100 + 200 < b.bytes);  // retired buffers together stay below the live one

  fa.limit = 1500;  // the doubled 2000 is refused, the exact 1200 granted
  const size_t before = fa.requests.size();
  CHECK(grow_buffer(b, 1200, fa, &out) == 0);
  CHECK(fa.requests.size() == before + 2 && fa.requests[before] == 2000 && fa.requests[before + 1] == 1200);
  CHECK(b.bytes == 1200 && b.retired.size() == 3);

  void* live = b.p;  // both requests refused: error status, entry unchanged
  CHECK(grow_buffer(b, 5000, fa, &out) == 7);
  CHECK(out == nullptr && b.p == live && b.bytes == 1200 && b.retired.size() == 3);

  GrowBuffer z;  // zero need on an empty entry: no allocation, null buffer
  CHECK(grow_buffer(z, 0, fa, &out) == 0 && out == nullptr && z.bytes == 0);

  miq::GrowBufferTable<int> t(3);
  GrowBuffer* e1 = t.find_or_add(1);
  GrowBuffer* e2 = t.find_or_add(2);
  GrowBuffer* e3 = t.find_or_add(3);
  CHECK(e1 && e2 && e3 && e1 != e2 && e2 != e3 && t.size() == 3);
  CHECK(t.find_or_add(4) == nullptr && t.size() == 3);  // full: a new key is refused
  CHECK(t.find_or_add(1) == e1 && t.find_or_add(3) == e3);  // existing keys still found
  FakeAlloc fb;
  CHECK(grow_buffer(*e2, 64, fb, &out) == 0 && t.find_or_add(2)->p == out);

  miq::GrowBufferTable<int> big(1000);  // entry addresses survive many additions
  GrowBuffer* e0 = big.find_or_add(0);
  for (int i = 1; i < 1000; ++i) big.find_or_add(i);
  CHECK(big.find_or_add(0) == e0 && big.size() == 1000);

  if (failures) return 1;
  std::printf("ok\n");
  return 0;
}

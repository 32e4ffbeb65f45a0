// Host unit test of the binning index guards (csrc/index_guard.hpp).
// Built and run by tests/test_index_guard.py with g++; prints "ok" on success.
#include <cstdio>
#include <cstdint>

#include "index_guard.hpp"

// The guards are constexpr, so their contract can also be checked at compile time.
constexpr bool in_range_passes() {
  bool bad = false;
  return gs::checked_index(5, 6, bad) == 5 && !bad;
}
constexpr bool past_end_is_replaced() {
  bool bad = false;
  return gs::checked_index(6, 6, bad) == 0 && bad;
}
static_assert(in_range_passes(), "an index below the count must pass unchanged");
static_assert(past_end_is_replaced(), "an index equal to the count must be replaced");

static int failures = 0;

static void expect(bool condition, const char* what) {
  if (!condition) {
    std::printf("FAIL: %s\n", what);
    ++failures;
  }
}

int main() {
  const int64_t cases[][3] = {
      // index, count, expected result (-1: flagged and replaced by 0)
      {0, 1, 0},       {0, 0, -1},           {-1, 10, -1},        {9, 10, 9},
      {10, 10, -1},    {2147483647, 2147483647, -1},  {2147483646, 2147483647, 2147483646},
      {int64_t(1) << 40, 100, -1}, {-(int64_t(1) << 40), 100, -1},
  };
  for (const auto& c : cases) {
    bool bad = false;
    const int got = gs::checked_index(c[0], c[1], bad);
    if (c[2] < 0) {
      expect(bad && got == 0, "an out-of-range index is flagged and replaced by 0");
    } else {
      expect(!bad && got == c[2], "an in-range index passes unchanged");
    }
  }
  // The flag is sticky: a later valid index does not clear it.
  bool bad = false;
  gs::checked_index(-5, 3, bad);
  gs::checked_index(1, 3, bad);
  expect(bad, "a raised flag stays raised");

  // Packed (tile id << bits | rank) keys give back their rank.
  expect(gs::packed_rank(0xABCDu << 12 | 0x123u, 12) == 0x123, "rank of a packed key");
  expect(gs::packed_rank(0xFFFFFFFFu, 32) == 0xFFFFFFFFll, "32 rank bits keep the whole key");
  expect(gs::packed_rank(0xFFFFFFFFu, 0) == 0, "0 rank bits give rank 0");
  // A corrupted rank past the pair count is caught by the range check.
  bool corrupt = false;
  const int rank = gs::checked_index(gs::packed_rank(7u << 10 | 1000u, 10), 1000, corrupt);
  expect(corrupt && rank == 0, "a packed rank equal to the pair count is flagged");

  expect(gs::kBinOverflow == 1u && gs::kBinBadIndex == 2u, "status bits match the C ABI");
  if (failures == 0) std::printf("ok\n");
  return failures == 0 ? 0 : 1;
}

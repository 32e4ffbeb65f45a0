// Range checks on indices that come out of a sort.
//
// The binning consumers dereference what the radix sorts produce: depth
// ranks become pair indices through `order`, and pair indices address the
// tile rectangles and, through the point list, every compositor gather. A
// sort that produced a stale or out-of-range index would otherwise read
// out of bounds. checked_index substitutes index 0 (a valid pair whenever
// there is one) and records the violation, so a broken sort gives wrong
// tiles and a raised flag instead of a memory fault.
//
// Plain constexpr functions: hipcc compiles them for the device, and the
// host unit test (tests/test_index_guard.py) compiles this header with g++.
#pragma once

#include <cstdint>

namespace gs {

// Status bits of the binning flag word (bit 0 is the capacity overflow).
constexpr uint32_t kBinOverflow = 1u;
constexpr uint32_t kBinBadIndex = 2u;

// `index` when 0 <= index < count; otherwise 0, with `bad` set.
constexpr int checked_index(int64_t index, int64_t count, bool& bad) {
  const bool ok = index >= 0 && index < count;
  if (!ok) bad = true;
  return ok ? static_cast<int>(index) : 0;
}

// Low `bits` bits of a packed (tile id, depth rank) key: the depth rank.
constexpr int64_t packed_rank(uint32_t key, int bits) {
  return bits >= 32 ? int64_t(key) : int64_t(key & ((1u << bits) - 1u));
}

}  // namespace gs

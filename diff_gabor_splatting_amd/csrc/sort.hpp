// Stable LSD radix sort of (key, int32 value) pairs, shared by the public
// 64-bit sort entry point and the depth-first binning pipeline.
#pragma once

#include "common.hpp"

namespace gs {

// Scratch bytes of radix_sort<Key> over m pairs.
size_t radix_sort_workspace_bytes(int64_t m, int key_bytes);

// Sorts on key bits [begin_bit, end_bit); Key is uint32_t or uint64_t.
// Null values_in and values_out sort the keys alone.
// Outputs must not alias inputs; the workspace is radix_sort_workspace_bytes.
// With `live` (a device int64), only the first min(*live, m) pairs are
// sorted; m is then the capacity the launches are sized for.
template <typename Key>
int radix_sort(const Key* keys_in, Key* keys_out, const int* values_in, int* values_out,
               int64_t m, int begin_bit, int end_bit, void* workspace, hipStream_t stream,
               const int64_t* live = nullptr);

}  // namespace gs

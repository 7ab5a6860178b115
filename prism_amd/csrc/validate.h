// Debug-mode work-list checks of the attention entry points (validate.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

// PRISM_DEBUG in the environment ("0" off, anything else on), else the build
// default PRISM_DEBUG_DEFAULT
bool prism_debug_enabled();

// Copies (start, len, cols) of `rows` device lists and, if given, the
// tile masks to the host (synchronising `stream`; every copy is first
// checked to lie inside the device allocation that holds it) and checks
// them: lengths in [0, ntiles], entries (entry >> 3 for
// pair unions) strictly ascending in [0, ntiles), union entries flagged for a
// tile of the pair and partial exactly where the tile mask is not full.
int prism_debug_check_lists(const char* who, const int64_t* start_d, const int32_t* len_d, const int32_t* cols_d,
                            int64_t rows, int64_t ntiles, int unions, const uint64_t* tile_masks_d,
                            hipStream_t stream);

// Copies pairmap ([heads, tiles_per_head]) and order ([n_order]) to the host,
// each if given, and checks that pairmap is a permutation of each head's
// tiles and order one of [0, n_order).
int prism_debug_check_maps(const char* who, const int32_t* pairmap_d, int64_t heads, int64_t tiles_per_head,
                           const int32_t* order_d, int64_t n_order, hipStream_t stream);

#define PRISM_DEBUG_CHECK(call)      \
  do {                               \
    const int _rc = (call);          \
    if (_rc != PRISM_OK) return _rc; \
  } while (0)

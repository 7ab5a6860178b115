// Work-list validation (host code; the debug mode of the attention entry
// points).
//
// The attention kernels index K/V (or Q/dO) tiles straight from their work
// lists and take their pairs from `pairmap` and `order`; a corrupt list would
// make them read outside the operands.  prism_check_lists and
// prism_check_launch_maps state every invariant the kernels rely on and check
// it on host copies.  With PRISM_DEBUG=1 in the environment (or a library
// built with PRISM_DEBUG_DEFAULT=1, unless PRISM_DEBUG=0), prism_bsa_fwd,
// prism_bsa_bwd_dkdv, prism_bsa_bwd_dq and prism_pair_union copy their lists
// to the host (a synchronisation on the call's stream) and check them before
// anything is launched: a violation returns PRISM_EINVAL naming the first bad
// row and entry, and no kernel runs.  No counterpart in the reference, whose
// Triton kernels read the lists unchecked.
#include <stdlib.h>
#include <string.h>

#include <vector>

#include "common.h"
#include "validate.h"

#ifndef PRISM_DEBUG_DEFAULT
#define PRISM_DEBUG_DEFAULT 0
#endif

namespace {

// n elements from dev, after checking that they lie inside the device
// allocation that holds dev (so that the copy itself cannot fault)
template <class T>
int to_host(std::vector<T>& out, const T* dev, int64_t n, hipStream_t stream, const char* who, const char* what) {
  out.clear();
  if (n <= 0) return PRISM_OK;
  void* base = nullptr;
  size_t size = 0;
  hipError_t e = hipMemGetAddressRange(&base, &size, (void*)dev);
  if (e != hipSuccess || base == nullptr) {
    prism_set_error("%s: debug check: %s is not device memory (%s)", who, what, hipGetErrorString(e));
    return PRISM_EINVAL;
  }
  const uint64_t avail = (uint64_t)((const char*)base + size - (const char*)dev) / sizeof(T);
  PRISM_REQUIRE((uint64_t)n <= avail, "%s: %s: %lld elements needed, %llu left in their allocation", who, what,
                (long long)n, (unsigned long long)avail);
  out.resize((size_t)n);
  e = hipMemcpyAsync(out.data(), dev, (size_t)n * sizeof(T), hipMemcpyDeviceToHost, stream);
  if (e == hipSuccess) e = hipStreamSynchronize(stream);
  if (e != hipSuccess) {
    prism_set_error("%s: debug check: copying %s to the host failed: %s", who, what, hipGetErrorString(e));
    return PRISM_EHIP;
  }
  return PRISM_OK;
}

int check_lists(const char* who, const int64_t* start, const int32_t* len, const int32_t* cols, int64_t rows,
                int64_t ncols, int64_t ntiles, int unions, const uint64_t* tile_masks) {
  PRISM_REQUIRE(rows >= 0 && ncols >= 0 && ntiles >= 1, "%s: bad list geometry (rows %lld, entries %lld, tiles %lld)",
                who, (long long)rows, (long long)ncols, (long long)ntiles);
  PRISM_REQUIRE(rows == 0 || (start && len), "%s: null list pointer", who);
  for (int64_t r = 0; r < rows; ++r) {
    const int64_t s = start[r], n = len[r];
    PRISM_REQUIRE(n >= 0 && n <= ntiles, "%s: row %lld has length %lld outside [0, %lld]", who, (long long)r,
                  (long long)n, (long long)ntiles);
    PRISM_REQUIRE(s >= 0 && s + n <= ncols, "%s: row %lld entries [%lld, %lld) outside the %lld list entries", who,
                  (long long)r, (long long)s, (long long)(s + n), (long long)ncols);
    if (n > 0) PRISM_REQUIRE(cols, "%s: null entry pointer", who);
    int64_t prev = -1;
    for (int64_t i = 0; i < n; ++i) {
      const int32_t e = cols[s + i];
      // unions: 1 = pair entries (tile << 3 | partial << 2 | 2 member bits),
      // 2 = quad entries (tile << 5 | partial << 4 | 4 member bits)
      const int mbits = unions == 2 ? 4 : 2;
      const int64_t t = unions ? (int64_t)(e >> (mbits + 1)) : (int64_t)e;
      PRISM_REQUIRE(e >= 0 && t < ntiles, "%s: row %lld entry %lld names tile %lld outside [0, %lld)", who,
                    (long long)r, (long long)i, (long long)t, (long long)ntiles);
      PRISM_REQUIRE(t > prev, "%s: row %lld entry %lld (tile %lld) is not above the previous tile %lld", who,
                    (long long)r, (long long)i, (long long)t, (long long)prev);
      prev = t;
      if (unions) {
        PRISM_REQUIRE((e & ((1 << mbits) - 1)) != 0, "%s: row %lld entry %lld (tile %lld) belongs to no tile of its %s",
                      who, (long long)r, (long long)i, (long long)t, unions == 2 ? "quad" : "pair");
        const bool partial = (e & (1 << mbits)) != 0;
        const bool want = tile_masks != nullptr && tile_masks[t] != ~0ull;
        PRISM_REQUIRE(partial == want, "%s: row %lld entry %lld: tile %lld is flagged %s but its key mask is %s", who,
                      (long long)r, (long long)i, (long long)t, partial ? "partial" : "full",
                      tile_masks == nullptr ? "absent" : want ? "partial" : "full");
      }
    }
  }
  return PRISM_OK;
}

int check_maps(const char* who, const int32_t* pairmap, int64_t heads, int64_t tiles_per_head, const int32_t* order,
               int64_t n_order) {
  if (pairmap) {
    PRISM_REQUIRE(heads >= 1 && tiles_per_head >= 2 && tiles_per_head % 2 == 0,
                  "%s: bad pairmap geometry (%lld heads of %lld tiles)", who, (long long)heads,
                  (long long)tiles_per_head);
    std::vector<uint8_t> seen((size_t)tiles_per_head);
    for (int64_t h = 0; h < heads; ++h) {
      memset(seen.data(), 0, seen.size());
      const int32_t* m = pairmap + h * tiles_per_head;
      for (int64_t i = 0; i < tiles_per_head; ++i) {
        PRISM_REQUIRE(m[i] >= 0 && m[i] < tiles_per_head,
                      "%s: pairmap of head %lld slot %lld names tile %d outside [0, %lld)", who, (long long)h,
                      (long long)i, m[i], (long long)tiles_per_head);
        PRISM_REQUIRE(!seen[m[i]], "%s: pairmap of head %lld names tile %d twice", who, (long long)h, m[i]);
        seen[m[i]] = 1;
      }
    }
  }
  if (order) {
    PRISM_REQUIRE(n_order >= 1, "%s: empty launch order", who);
    std::vector<uint8_t> seen((size_t)n_order, 0);
    for (int64_t i = 0; i < n_order; ++i) {
      PRISM_REQUIRE(order[i] >= 0 && order[i] < n_order, "%s: launch order slot %lld names pair %d outside [0, %lld)",
                    who, (long long)i, order[i], (long long)n_order);
      PRISM_REQUIRE(!seen[order[i]], "%s: launch order names pair %d twice", who, order[i]);
      seen[order[i]] = 1;
    }
  }
  return PRISM_OK;
}

}  // namespace

bool prism_debug_enabled() {
  const char* s = getenv("PRISM_DEBUG");
  if (s && *s) return strcmp(s, "0") != 0;
  return PRISM_DEBUG_DEFAULT != 0;
}

int prism_debug_check_lists(const char* who, const int64_t* start_d, const int32_t* len_d, const int32_t* cols_d,
                            int64_t rows, int64_t ntiles, int unions, const uint64_t* tile_masks_d,
                            hipStream_t stream) {
  std::vector<int64_t> start;
  std::vector<int32_t> len, cols;
  std::vector<uint64_t> masks;
  int rc = to_host(start, start_d, rows, stream, who, "list starts");
  if (rc == PRISM_OK) rc = to_host(len, len_d, rows, stream, who, "list lengths");
  if (rc != PRISM_OK) return rc;
  // the entries' extent: the end of the furthest row (the C-ABI does not
  // carry the entries' size; to_host checks it against their allocation)
  int64_t extent = 0;
  for (int64_t r = 0; r < rows; ++r) {
    PRISM_REQUIRE(start[r] >= 0 && len[r] >= 0 && len[r] <= ntiles,
                  "%s: row %lld has start %lld and length %d (tiles %lld)", who, (long long)r, (long long)start[r],
                  len[r], (long long)ntiles);
    if (start[r] + len[r] > extent) extent = start[r] + len[r];
  }
  rc = to_host(cols, cols_d, extent, stream, who, "list entries");
  if (rc == PRISM_OK && tile_masks_d) rc = to_host(masks, tile_masks_d, ntiles, stream, who, "tile masks");
  if (rc != PRISM_OK) return rc;
  return check_lists(who, start.data(), len.data(), cols.data(), rows, extent, ntiles, unions,
                     tile_masks_d ? masks.data() : nullptr);
}

int prism_debug_check_maps(const char* who, const int32_t* pairmap_d, int64_t heads, int64_t tiles_per_head,
                           const int32_t* order_d, int64_t n_order, hipStream_t stream) {
  std::vector<int32_t> pairmap, order;
  int rc = PRISM_OK;
  if (pairmap_d) rc = to_host(pairmap, pairmap_d, heads * tiles_per_head, stream, who, "pairmap");
  if (rc == PRISM_OK && order_d) rc = to_host(order, order_d, n_order, stream, who, "launch order");
  if (rc != PRISM_OK) return rc;
  return check_maps(who, pairmap_d ? pairmap.data() : nullptr, heads, tiles_per_head,
                    order_d ? order.data() : nullptr, n_order);
}

extern "C" {

int prism_check_lists(const int64_t* start, const int32_t* len, const int32_t* cols, int64_t rows, int64_t ncols,
                      int64_t ntiles, int unions, const uint64_t* tile_masks) {
  return check_lists("prism_check_lists", start, len, cols, rows, ncols, ntiles, unions, tile_masks);
}

int prism_check_launch_maps(const int32_t* pairmap, int64_t heads, int64_t tiles_per_head, const int32_t* order,
                            int64_t n_order) {
  return check_maps("prism_check_launch_maps", pairmap, heads, tiles_per_head, order, n_order);
}

}  // extern "C"

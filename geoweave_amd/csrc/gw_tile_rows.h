// Row arithmetic of the masked dense kernels' 64-row tile loads, kept free of HIP headers so
// that the same code is compiled for the GPU kernels and by a host-side test.
//
// A tile of 64 rows starting at row k0 (a multiple of 64) of an n-row operand (n >= 1) is
// loaded as rows srow and srow + 32 per thread (srow < 32). Rows past the last one read row
// n - 1. Addresses are a uniform base row plus a 32-bit lane offset (row offset times the row
// stride, a 24-bit multiply), so the base is min(k0, n - 1): padded query or key blocks can
// start at or past n, and an offset taken from k0 there would be negative.
#pragma once

#include <stdint.h>

namespace gw {

struct TileRows {
  int base;     // first row of the tile's address range
  uint32_t r0;  // row offset of row srow from base, in [0, 63]
  uint32_t r1;  // row offset of row srow + 32 from base, in [0, 63]
};

constexpr int tile_imin(int a, int b) { return a < b ? a : b; }

constexpr TileRows tile_rows(int k0, int srow, int n) {
  return TileRows{tile_imin(k0, n - 1), (uint32_t)(tile_imin(k0 + srow, n - 1) - tile_imin(k0, n - 1)),
                  (uint32_t)(tile_imin(k0 + srow + 32, n - 1) - tile_imin(k0, n - 1))};
}

}  // namespace gw

// Layout constants shared by the re-tiling kernels and the decode kernels.
#pragma once

#include <stdint.h>

namespace lsq {

// Tiled INT4 decode layout. The weight matrix is cut into tiles of kTileN rows by
// kTileK columns (one 128-wide quantization group), stored tile after tile in
// (row-tile, k-tile) order, kTileBytes contiguous bytes each. Inside a tile, lane l of
// a 64-lane wavefront owns bytes [16 l, 16 l + 16): row r = l & 15 and columns
// [32 (l >> 4), 32 (l >> 4) + 32) of the tile. Dword d of those 16 bytes holds the 8
// columns c0 = 32 (l >> 4) + 8 d + e, e = 0..7, one per nibble; nibble position p holds
// column offset e = tiled_nibble_k(p), so that (nibble p, nibble p + 4) is the adjacent
// column pair (2p, 2p + 1) and one AND-OR with a magic exponent turns it into a packed
// bf16/fp16 pair in the same order as the activations.
constexpr int kTileN = 16;
constexpr int kTileK = 128;
constexpr int kTileBytes = kTileN * kTileK / 2;

__host__ __device__ constexpr int tiled_nibble_k(int p) { return p < 4 ? 2 * p : 2 * (p - 4) + 1; }

// Tiled INT8 decode layout: the same 16-row x 128-column tiles in (row-tile, k-tile)
// order, kTileBytes8 contiguous bytes each, made of two 1 KB halves j = 0, 1. Byte
// j * 1024 + 16 l + b of a tile is W[16 rt + (l & 15)][128 kt + 32 (l >> 4) + 16 j + b],
// so each 64-lane wavefront load reads 1 KB contiguous and lane l ends up with the 32
// consecutive columns [32 (l >> 4), 32 (l >> 4) + 32) of row l & 15 of the tile.
constexpr int kTileBytes8 = kTileN * kTileK;

}  // namespace lsq

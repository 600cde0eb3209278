// Launch geometry and address arithmetic of the GEMV kernel, shared by the
// device code and by a host-side bounds checker (tests/test_gemv_addressing.py
// compiles this header with g++ and enumerates every load the kernel issues).
//
// Layout: W is row-major [R, K] in 16-byte chunks (kElems values per chunk,
// nchunks = K / kElems per row).  A wave owns 8-row tiles; lane (r = lane/8,
// j = lane%8) reads chunk (batch*kUnroll + u)*8 + j of row tile*8 + r.
// Every offset below is non-negative and in bounds: rows past R re-read row
// R-1 and chunks past the row end re-read the row's last chunk.
#pragma once

#include <cstddef>
#include <cstdint>

#ifndef __HIPCC__
#define CPI_HD
#else
#define CPI_HD __host__ __device__
#endif

namespace cpi {

constexpr int kChunkCols = 8;                 // 16-byte chunks per row per step
constexpr int kTileRows = 8;                  // rows per wave tile (64 lanes / 8)
constexpr int kWavesPerBlock = 4;
constexpr int kUnroll = 4;                    // steps per batch

struct GemvGeom {
  int R, K, elems;        // rows, columns, values per 16-byte chunk
  int ks;                 // K-segments per tile (waves cooperating on a tile)
  int grid;               // workgroups
  int tpw;                // tiles per workgroup iteration = 4 / ks
  int tiles, nchunks, steps, nbt, nbs, groups;
  uint32_t row_bytes;
};

CPI_HD inline GemvGeom make_geom(int R, int K, int elems, int ks, int grid) {
  GemvGeom g;
  g.R = R;
  g.K = K;
  g.elems = elems;
  g.ks = ks;
  g.grid = grid;
  g.tpw = kWavesPerBlock / ks;
  g.tiles = (R + kTileRows - 1) / kTileRows;
  g.nchunks = K / elems;
  g.steps = (g.nchunks + kChunkCols - 1) / kChunkCols;
  g.nbt = (g.steps + kUnroll - 1) / kUnroll;
  g.nbs = (g.nbt + ks - 1) / ks;
  g.groups = (g.tiles + g.tpw - 1) / g.tpw;
  g.row_bytes = static_cast<uint32_t>(K) * 16u / static_cast<uint32_t>(elems);
  return g;
}

// Host launch plan: K-split so the launch has >= ~2048 waves when possible.
inline void plan_launch(int R, int K, int elems, int max_blocks, int force_ks, int* ks_out,
                        int* grid_out) {
  const int tiles = (R + kTileRows - 1) / kTileRows;
  const int steps = (K / elems + kChunkCols - 1) / kChunkCols;
  const int nbt = (steps + kUnroll - 1) / kUnroll;
  int ks = 1;
  if (force_ks > 0) ks = force_ks;
  else if (tiles < 1024 && nbt >= 4) ks = 4;
  else if (tiles < 1536 && nbt >= 2) ks = 2;
  if (ks > nbt) ks = nbt >= 4 ? 4 : (nbt >= 2 ? 2 : 1);
  const int tpw = kWavesPerBlock / ks;
  int grid = (tiles + tpw - 1) / tpw;
  if (grid > max_blocks) grid = max_blocks;
  if (grid < 1) grid = 1;
  *ks_out = ks;
  *grid_out = grid;
}

// Number of tile groups workgroup `block` processes, and the last one.
CPI_HD inline int my_groups(const GemvGeom& g, int block) {
  return g.groups > block ? (g.groups - block + g.grid - 1) / g.grid : 0;
}

// Wave-uniform description of one batch position.
struct BatchPos {
  int tile;    // tile index actually read (clamped into range)
  int row0;    // first row of the tile
  int rmax;    // last valid row offset inside the tile (< 8 only for the last tile)
  int cbase;   // first chunk of the batch (may be >= nchunks for an empty batch)
  bool full;   // all chunks of the batch are < nchunks
};

// Batch (group gpos, batch bb of the wave's segment); positions past the
// workgroup's work are clamped to its last batch (their loads are discarded).
CPI_HD inline BatchPos batch_pos(const GemvGeom& g, int block, int wave, int gpos, int bb) {
  const int mg = my_groups(g, block);
  const int last_g = block + (mg > 0 ? mg - 1 : 0) * g.grid;
  if (gpos > last_g) {
    gpos = last_g;
    bb = g.nbs - 1;
  }
  int t = gpos * g.tpw + wave / g.ks;
  if (t >= g.tiles) t = g.tiles - 1;
  BatchPos b;
  b.tile = t;
  b.row0 = t * kTileRows;
  const int last = g.R - 1 - b.row0;
  b.rmax = last < kTileRows - 1 ? last : kTileRows - 1;
  b.cbase = ((wave % g.ks) * g.nbs + bb) * kUnroll * kChunkCols;
  b.full = b.cbase + kUnroll * kChunkCols <= g.nchunks;
  return b;
}

// Chunk index (within its row) that lane (r, j) reads for step u of batch b.
CPI_HD inline int lane_chunk(const GemvGeom& g, const BatchPos& b, int j, int u) {
  const int c = b.cbase + u * kChunkCols + j;
  return c < g.nchunks ? c : g.nchunks - 1;
}

CPI_HD inline int lane_row(const BatchPos& b, int r) { return b.row0 + (r < b.rmax ? r : b.rmax); }

// Byte offset of the 16-byte weight chunk, and element index of its fp16
// group scale (I4G32: one scale per chunk).
CPI_HD inline size_t weight_offset(const GemvGeom& g, const BatchPos& b, int r, int j, int u) {
  return static_cast<size_t>(lane_row(b, r)) * g.row_bytes + static_cast<size_t>(lane_chunk(g, b, j, u)) * 16u;
}
CPI_HD inline size_t scale_index(const GemvGeom& g, const BatchPos& b, int r, int j, int u) {
  return static_cast<size_t>(lane_row(b, r)) * static_cast<size_t>(g.nchunks) +
         static_cast<size_t>(lane_chunk(g, b, j, u));
}

}  // namespace cpi

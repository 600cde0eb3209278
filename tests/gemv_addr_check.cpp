// Host replay of the GEMV kernel's load/compute schedule (cpi_amd/csrc/gemv_plan.hpp):
// every weight / scale address must be in bounds and every (row, chunk) pair of
// the matrix must be accumulated exactly once.  Usage: gemv_addr_check R K elems max_blocks force_ks
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "../cpi_amd/csrc/gemv_plan.hpp"

using namespace cpi;

int main(int argc, char** argv) {
  if (argc < 6) return 2;
  const int R = atoi(argv[1]), K = atoi(argv[2]), elems = atoi(argv[3]);
  const int max_blocks = atoi(argv[4]), force_ks = atoi(argv[5]);
  int ks = 0, grid = 0;
  plan_launch(R, K, elems, max_blocks, force_ks, &ks, &grid);
  const GemvGeom g = make_geom(R, K, elems, ks, grid);
  const size_t wbytes = static_cast<size_t>(R) * g.row_bytes;
  const size_t nscales = static_cast<size_t>(R) * g.nchunks;
  std::vector<int> hits(static_cast<size_t>(R) * g.nchunks, 0);
  long loads = 0;
  for (int block = 0; block < grid; ++block) {
    const int total = my_groups(g, block) * g.nbs;
    for (int wave = 0; wave < kWavesPerBlock; ++wave) {
      // positions in kernel order: (block, 0) and its successors
      int gp = block, bb = 0;
      for (int it = 0; it < total + 2 && total > 0; ++it) {
        const BatchPos bp = batch_pos(g, block, wave, gp, bb);
        for (int lane = 0; lane < 64; ++lane) {
          const int r = lane / kChunkCols, j = lane % kChunkCols;
          for (int u = 0; u < kUnroll; ++u) {
            const size_t off = weight_offset(g, bp, r, j, u);
            const size_t si = scale_index(g, bp, r, j, u);
            ++loads;
            if (off + 16 > wbytes || si >= nscales) {
              printf("OOB R=%d K=%d block=%d wave=%d it=%d lane=%d u=%d off=%zu/%zu si=%zu/%zu\n", R, K,
                     block, wave, it, lane, u, off, wbytes, si, nscales);
              return 1;
            }
            // accumulation: only steps < total, real tiles, real rows, real chunks
            const int t = gp * g.tpw + wave / g.ks;
            const int c = bp.cbase + u * kChunkCols + j;
            const int row = t * kTileRows + r;
            if (it < total && t < g.tiles && row < R && c < g.nchunks) {
              if (bp.tile != t || (bp.full == false && c >= g.nchunks)) {
                printf("schedule mismatch\n");
                return 1;
              }
              ++hits[static_cast<size_t>(row) * g.nchunks + c];
            }
          }
        }
        if (++bb == g.nbs) { bb = 0; gp += grid; }
      }
    }
  }
  for (size_t i = 0; i < hits.size(); ++i)
    if (hits[i] != 1) {
      printf("coverage R=%d K=%d ks=%d grid=%d: row %zu chunk %zu hit %d times\n", R, K, ks, grid,
             i / g.nchunks, i % g.nchunks, hits[i]);
      return 1;
    }
  printf("ok R=%d K=%d elems=%d ks=%d grid=%d loads=%ld\n", R, K, elems, ks, grid, loads);
  return 0;
}

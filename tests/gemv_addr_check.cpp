// Host replay of the GEMV kernel's load/compute schedule (cpi_amd/csrc/gemv_plan.hpp):
// every weight / scale address (row-major and blocked group scales) must be in
// bounds and every (row, chunk) pair of the matrix must be accumulated exactly
// once, with its own scale.
// Usage: gemv_addr_check R K elems force_shape force_ks
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "../cpi_amd/csrc/gemv_plan.hpp"

using namespace cpi;

int main(int argc, char** argv) {
  if (argc < 6) return 2;
  const int R = atoi(argv[1]), K = atoi(argv[2]), elems = atoi(argv[3]);
  const int force_shape = atoi(argv[4]), force_ks = atoi(argv[5]);
  const GemvPlan g = plan_launch(R, K, elems, force_shape, force_ks);
  if (g.nr * g.pp > kMaxLoads || g.rb % kTileRows != 0 || g.rb > kWavesPerBlock * 8) {
    printf("bad plan nr=%d pp=%d rb=%d\n", g.nr, g.pp, g.rb);
    return 1;
  }
  const size_t wbytes = static_cast<size_t>(R) * g.row_bytes;
  const size_t nscales = static_cast<size_t>(R) * g.nchunks;
  const size_t nblocked = blocked_scale_elems(R, g.nchunks);
  std::vector<int> hits(static_cast<size_t>(R) * g.nchunks, 0);
  long loads = 0;
  for (int block = 0; block < g.grid; ++block)
    for (int wave = 0; wave < kWavesPerBlock; ++wave) {
      const int rs = wave / g.ks, sg = wave % g.ks;
      for (int grp = 0; grp < g.ng; ++grp)
        for (int q = 0; q < g.pp; ++q) {
          const int pass_u = plan_pass(g, sg, grp, q);
          const int pass = clamp_pass(g, sg, pass_u);
          for (int lane = 0; lane < 64; ++lane) {
            const int c = clamp_chunk(g, pass, lane);
            // blocked scales: one load of nr elements from the row group's first row
            const int row0 = plan_row(g, block, rs, 0);
            const size_t sb = scale_block_index(g, clamp_row_group(g, row0, g.nr), c);
            if (sb + g.nr > nblocked || sb % g.nr != 0) {
              printf("blocked scale load OOB/misaligned R=%d K=%d block=%d wave=%d lane=%d at %zu/%zu\n", R, K, block,
                     wave, lane, sb, nblocked);
              return 1;
            }
            for (int i = 0; i < g.nr; ++i) {
              const int row_u = plan_row(g, block, rs, i);
              const int row = clamp_row(g, row_u);
              const size_t off = weight_offset(g, row, c);
              const size_t si = scale_index(g, row, c);
              ++loads;
              if (off + 16 > wbytes || si >= nscales || c < 0 || row < 0) {
                printf("OOB R=%d K=%d block=%d wave=%d grp=%d q=%d lane=%d i=%d off=%zu/%zu si=%zu/%zu\n", R, K,
                       block, wave, grp, q, lane, i, off, wbytes, si, nscales);
                return 1;
              }
              // accumulated by the kernel: valid pass of the segment, real chunk, real row
              const int cu = pass_u * kPassChunks + lane;
              if (pass_valid(g, sg, pass_u) && cu < g.nchunks && row_u < R) {
                if (cu != c || row_u != row) {
                  printf("clamped load accumulated\n");
                  return 1;
                }
                if (sb + i != scale_block_index(g, row, c)) {
                  printf("blocked scale of row %d chunk %d read from the wrong element\n", row, c);
                  return 1;
                }
                ++hits[static_cast<size_t>(row) * g.nchunks + c];
              }
            }
          }
        }
    }
  for (size_t i = 0; i < hits.size(); ++i)
    if (hits[i] != 1) {
      printf("coverage R=%d K=%d nr=%d pp=%d ks=%d: row %zu chunk %zu hit %d times\n", R, K, g.nr, g.pp, g.ks,
             i / g.nchunks, i % g.nchunks, hits[i]);
      return 1;
    }
  printf("ok R=%d K=%d elems=%d nr=%d pp=%d ks=%d ng=%d grid=%d loads=%ld\n", R, K, elems, g.nr, g.pp, g.ks, g.ng,
         g.grid, loads);
  return 0;
}

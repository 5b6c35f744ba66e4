// Host-only: pet::build_edges on a structure read from a text file, the
// edges written back as text (centre neighbour sx sy sz reverse), for
// tests/test_neighbors.py to compare with an independent brute force.
//   neighbors_dump IN OUT cutoff
// IN: N, then 3 cell rows, then N lines "x y z".
#include <cstdio>
#include <cstdlib>

#include "pet/model.hpp"

int main(int argc, char** argv) {
  if (argc != 4) return 2;
  FILE* f = std::fopen(argv[1], "r");
  if (!f) return 3;
  int N = 0;
  if (std::fscanf(f, "%d", &N) != 1) return 4;
  pet::System s;
  for (int r = 0; r < 3; ++r)
    for (int c = 0; c < 3; ++c)
      if (std::fscanf(f, "%lf", &s.cell[r][c]) != 1) return 4;
  s.positions.resize(N);
  s.numbers.assign(N, 6);
  for (int n = 0; n < N; ++n)
    for (int c = 0; c < 3; ++c)
      if (std::fscanf(f, "%lf", &s.positions[n][c]) != 1) return 4;
  std::fclose(f);
  const pet::HostEdges e = pet::build_edges(s, std::atof(argv[3]), 0.5, 1);
  FILE* o = std::fopen(argv[2], "w");
  if (!o) return 5;
  for (size_t k = 0; k < e.center.size(); ++k)
    std::fprintf(o, "%d %d %d %d %d %d\n", e.center[k], e.neigh[k], e.shift[3 * k], e.shift[3 * k + 1],
                 e.shift[3 * k + 2], e.reverse[k]);
  std::fclose(o);
  return 0;
}

// Host driver for the weight-gradient K-tile window arithmetic (ktile.h):
// prints "kt offset bytes" for every K-tile of one group (and one past its
// end), then the window of a dead pipeline slot.  Built and run by
// tests/test_ktile_window.py with the host compiler.
#include <cstdio>
#include <cstdlib>

#include "ktile.h"

int main(int argc, char** argv) {
  if (argc != 3) return 2;
  const unsigned long long rows = std::strtoull(argv[1], nullptr, 10);
  const unsigned row_bytes = (unsigned)std::strtoul(argv[2], nullptr, 10);
  const unsigned long long group_bytes = rows * row_bytes;
  const int nk = (int)((rows + pmx::kKTileRows - 1) / pmx::kKTileRows);
  for (int kt = 0; kt <= nk; ++kt) {
    const pmx::KTileWindow w = pmx::ktile_window(group_bytes, row_bytes, kt, true);
    std::printf("%d %llu %llu\n", kt, (unsigned long long)w.offset, (unsigned long long)w.bytes);
  }
  const pmx::KTileWindow d = pmx::ktile_window(group_bytes, row_bytes, nk / 2, false);
  std::printf("dead %llu %llu\n", (unsigned long long)d.offset, (unsigned long long)d.bytes);
  return 0;
}

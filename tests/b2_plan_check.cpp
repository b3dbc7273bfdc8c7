// Checks the concatenated row plan of the column-split backward
// (laplacianformer_amd/csrc/b2_plan.h) over many source lengths and batch
// sizes, decoding each wave entry the way laplace_bwd2.hip does: every row of
// a slice is taken exactly once, by a wave of the workgroup whose range holds
// it; waves stay within their source and within b2_max_wave_rows(12) rows;
// their LDS rows are disjoint and inside the kB2MaxRows-row tile; a wave
// without rows points at a valid row. Prints "ok <planned> <shapes>" or the
// first violation, and exits non-zero on one.
#include <cstdio>
#include <vector>

#include "../laplacianformer_amd/csrc/b2_plan.h"

using namespace lfamd;

static int check(const std::vector<int64_t>& L, int64_t slices, int cus, int& planned) {
  const int nsrc = (int)L.size();
  const int nx = b2_cat_nx(nsrc, L.data(), slices, cus);
  if (nx == 0) return 0;
  std::vector<uint32_t> wv(kB2CatSlots * 12, 0xffffffffu);
  if (!b2_cat_tables(nsrc, L.data(), nx, wv.data())) return 0;
  ++planned;
  int64_t tot = 0;
  std::vector<int64_t> base(nsrc, 0);
  for (int i = 0; i < nsrc; ++i) {
    base[i] = tot;
    tot += L[i];
  }
  std::vector<int> cover(tot, 0);
  for (int x = 0; x < nx; ++x) {
    const int64_t lo = x * tot / nx, hi = (x + 1) * tot / nx;
    if (hi - lo > kB2MaxRows) return printf("workgroup %d of %lld rows\n", x, (long long)(hi - lo)), 1;
    std::vector<int> lds(kB2MaxRows, 0);
    for (int w = 0; w < 12; ++w) {
      const uint32_t e = wv[x * 12 + w];
      const int si = (int)(e & 3u), rows = (int)((e >> 2) & 127u), l0 = (int)((e >> 9) & 1023u), st = (int)(e >> 19);
      if (si >= nsrc || st >= L[si] || rows > b2_max_wave_rows(12) || l0 + rows > kB2MaxRows)
        return printf("bad entry x=%d w=%d: src %d rows %d lds %d first %d\n", x, w, si, rows, l0, st), 1;
      for (int r = 0; r < rows; ++r) {
        if (lds[l0 + r]++) return printf("LDS row %d taken twice (x=%d)\n", l0 + r, x), 1;
        const int64_t g = base[si] + st + r;
        if (st + r >= L[si] || g < lo || g >= hi) return printf("row %lld outside workgroup %d\n", (long long)g, x), 1;
        cover[g]++;
      }
    }
  }
  for (int64_t g = 0; g < tot; ++g)
    if (cover[g] != 1) return printf("row %lld taken %d times\n", (long long)g, cover[g]), 1;
  return 0;
}

int main() {
  std::vector<std::vector<int64_t>> lens = {{49, 784, 784}, {784, 784, 49}, {65, 1, 200}, {130, 7}, {1, 1, 1},
                                            {1, 130, 49},   {300, 5},       {49, 3136, 3136}, {512, 512, 512},
                                            {1000, 3000},   {4096, 1},      {2, 3}};
  for (int a = 1; a <= 600; a += 37)
    for (int b = 1; b <= 900; b += 53) lens.push_back({a, b, (a * 7 + b) % 300 + 1});
  int planned = 0, shapes = 0;
  for (const auto& L : lens)
    for (int64_t slices : {1, 4, 32, 64, 128, 256, 1024})
      for (int cus : {256, 304}) {
        ++shapes;
        if (check(L, slices, cus, planned)) return 1;
      }
  // The attention layer's launch (K_mm, K_qm, K_km rows; 128 slices, 256 CUs):
  // four 404-row workgroups, K_mm's 49 rows on two waves of the youngest place.
  const int64_t layer[3] = {49, 784, 784};
  if (b2_cat_nx(3, layer, 128, 256) != 4) return printf("layer: nx %d\n", b2_cat_nx(3, layer, 128, 256)), 1;
  uint32_t wv[kB2CatSlots * 12];
  if (!b2_cat_tables(3, layer, 4, wv)) return printf("layer: no plan\n"), 1;
  int kmmWaves = 0, kmmRows = 0;
  for (int w = 0; w < 12; ++w)
    if ((wv[w] & 3u) == 0 && ((wv[w] >> 2) & 127u) > 0) {
      if (w < 8) return printf("layer: K_mm rows on wave %d\n", w), 1;
      ++kmmWaves;
      kmmRows += (int)((wv[w] >> 2) & 127u);
    }
  if (kmmWaves != 2 || kmmRows != 49) return printf("layer: K_mm on %d waves, %d rows\n", kmmWaves, kmmRows), 1;
  printf("ok %d %d\n", planned, shapes);
  return 0;
}

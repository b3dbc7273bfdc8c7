// Host-side row plan of the column-split backward (laplace_bwd2.hip): the row
// limits and per-place wave weights, and the concatenated plan of a launch over
// up to three row sources (B2Seg::cat). Plain C++ (no device code), so that a
// host compiler can build the plan alone.
#pragma once

#include <algorithm>
#include <cstdint>

namespace lfamd {

constexpr int kB2MaxRows = 512;  // most grad rows of one workgroup (staged in LDS at once)

// With 12 waves (waves w, w + 4, w + 8 share SIMD w % 4) the three places of a
// SIMD get kB2P0, kB2P1, kB2P2 parts of its rows: with an even split the
// youngest wave of each SIMD finished ~25 % after the others and then ran alone
// at half rate. (Per place, the middle wave runs its rows ~10 % faster than the
// oldest, but giving it more rows, 34 / 37 / 28, changed the kernel by < 0.2 %.)
constexpr int kB2P0 = 35, kB2P1 = 35, kB2P2 = 29, kB2PSum = 4 * (kB2P0 + kB2P1 + kB2P2);

// Most rows one wave of a WAVES-wave workgroup gets from the weighted split
// (floor(u1 n / S) - floor(u0 n / S) <= ceil((u1 - u0) n / S)).
constexpr int b2_max_wave_rows(int waves) {
  return waves == 12 ? (kB2MaxRows * (kB2P0 > kB2P1 ? (kB2P0 > kB2P2 ? kB2P0 : kB2P2) : (kB2P1 > kB2P2 ? kB2P1 : kB2P2)) +
                        kB2PSum - 1) / kB2PSum
                     : (kB2MaxRows + waves - 1) / waves;
}

constexpr int kB2CatSlots = 8;  // most workgroups per slice of a concatenated plan

// Wave table entry of a concatenated plan: source (bits 0-1), row count
// (2-8), first LDS row (9-18), first row within the source (19-31).
inline uint32_t b2_cat_entry(int src, int rows, int lds, int first) {
  return (uint32_t)src | (uint32_t)rows << 2 | (uint32_t)lds << 9 | (uint32_t)first << 19;
}

// Modelled duration of one SIMD's row work (M = 49, 12 waves) whose oldest,
// middle and youngest waves have r[0], r[1], r[2] rows: three busy waves
// issue at rate 1 and share it 35 : 35 : 29 (the weighted split that makes
// them end together), two at 0.864 (the measured 118 against 102 cycles per
// row of 8- and 12-wave workgroups) and one alone at 0.5, shared evenly.
inline double b2_simd_time(const int (&r)[3]) {
  double rem[3] = {(double)r[0], (double)r[1], (double)r[2]}, t = 0.0;
  const double w3[3] = {kB2P0 / 99.0, kB2P1 / 99.0, kB2P2 / 99.0};
  for (;;) {
    int act[3], na = 0;
    for (int i = 0; i < 3; ++i)
      if (rem[i] > 1e-9) act[na++] = i;
    if (na == 0) return t;
    double sh[3], dt = 1e300;
    for (int a = 0; a < na; ++a) {
      sh[a] = na == 3 ? w3[act[a]] : (na == 2 ? 0.864 : 0.5) / na;
      dt = std::min(dt, rem[act[a]] / sh[a]);
    }
    for (int a = 0; a < na; ++a) rem[act[a]] -= sh[a] * dt;
    t += dt;
  }
}

// Waves of one workgroup of a concatenated plan: the k pieces (source, first
// row, length) of its row range, in order, become the 12 wave table entries
// wv[0..11]. Each piece gets a run of waves, taken from the youngest places
// first (a short piece on the waves that get the fewest rows) and split over
// them by the kB2P weights; the counts and the order of the pieces are searched
// for the least modelled time of the slowest SIMD. A wave without rows points
// at its piece's first row. False when some wave would get more than
// b2_max_wave_rows(12) rows.
inline bool b2_cat_waves(int k, const int (&src)[3], const int (&start)[3], const int (&len)[3], uint32_t* wv) {
  static constexpr int kPref[12] = {8, 9, 10, 11, 4, 5, 6, 7, 0, 1, 2, 3};  // youngest places first
  auto units = [](int w) { return w < 4 ? kB2P0 : w < 8 ? kB2P1 : kB2P2; };
  double best = 1e300;
  int c[3] = {0, 0, 0};
  for (c[0] = 1; c[0] <= 12; ++c[0])
    for (c[1] = k > 1 ? 1 : 0; c[1] <= (k > 1 ? 12 : 0); ++c[1]) {
      c[2] = k > 2 ? 12 - c[0] - c[1] : 0;
      if (c[0] + c[1] + c[2] != 12 || (k > 2 && c[2] < 1)) continue;
      bool fits = true;
      for (int j = 0; j < k; ++j) fits = fits && c[j] <= std::max(1, len[j]);
      if (!fits) continue;
      int perm[3] = {0, 1, 2};
      do {
        int rows[12] = {}, first[12] = {}, from[12] = {}, pos = 0;
        for (int a = 0; a < k; ++a) {
          const int j = perm[a];
          int ws[12];
          for (int i = 0; i < c[j]; ++i) ws[i] = kPref[pos + i];
          pos += c[j];
          std::sort(ws, ws + c[j]);
          int tot = 0, cum = 0, prev = 0, off = start[j];
          for (int i = 0; i < c[j]; ++i) tot += units(ws[i]);
          for (int i = 0; i < c[j]; ++i) {
            cum += units(ws[i]);
            const int next = (int)((int64_t)cum * len[j] / tot);
            rows[ws[i]] = next - prev;
            from[ws[i]] = j;
            first[ws[i]] = rows[ws[i]] > 0 ? off : start[j];
            off += next - prev;
            prev = next;
          }
        }
        int mx = 0;
        for (int w = 0; w < 12; ++w) mx = std::max(mx, rows[w]);
        if (mx > b2_max_wave_rows(12)) continue;
        double cost = 0.0;
        for (int s = 0; s < 4; ++s) {
          const int r3[3] = {rows[s], rows[s + 4], rows[s + 8]};
          cost = std::max(cost, b2_simd_time(r3));
        }
        if (cost < best) {
          best = cost;
          int lds = 0;
          for (int w = 0; w < 12; ++w) {
            wv[w] = b2_cat_entry(src[from[w]], rows[w], rows[w] > 0 ? lds : 0, first[w]);
            lds += rows[w];
          }
        }
      } while (std::next_permutation(perm, perm + k));
    }
  return best < 1e300;
}

// Workgroups per slice of a concatenated plan for 2 or 3 sources of n[i] rows
// (the single-source rule for their total: at most kB2MaxRows rows each, one
// per CU where at least 8 rows each allow), or 0 when that is more than
// kB2CatSlots (or there is one source).
inline int b2_cat_nx(int nsrc, const int64_t* n, int64_t slices, int cus) {
  if (nsrc < 2 || nsrc > 3) return 0;
  int64_t tot = 0;
  for (int i = 0; i < nsrc; ++i) tot += n[i];
  const int64_t nx = std::max<int64_t>((tot + kB2MaxRows - 1) / kB2MaxRows,
                                       std::max<int64_t>(1, std::min<int64_t>(cus / std::max<int64_t>(slices, 1),
                                                                              (tot + 7) / 8)));
  return nx > kB2CatSlots || tot > (int64_t)kB2CatSlots * kB2MaxRows ? 0 : (int)nx;
}

// Wave tables wv[x * 12 + w] of the nx workgroups: workgroup x takes rows
// [x T / nx, (x + 1) T / nx) of the concatenated T = sum n[i] rows (source 0's,
// then 1's, then 2's). False when some workgroup has no fitting wave split.
inline bool b2_cat_tables(int nsrc, const int64_t* n, int nx, uint32_t* wv) {
  int64_t tot = 0;
  for (int i = 0; i < nsrc; ++i) tot += n[i];
  for (int x = 0; x < nx; ++x) {
    const int64_t a = (int64_t)x * tot / nx, b = (int64_t)(x + 1) * tot / nx;
    int k = 0, src[3] = {}, start[3] = {}, len[3] = {};
    int64_t s0 = 0;
    for (int i = 0; i < nsrc; ++i) {
      const int64_t lo = std::max(a, s0), hi = std::min(b, s0 + n[i]);
      if (hi > lo) {
        src[k] = i;
        start[k] = (int)(lo - s0);
        len[k] = (int)(hi - lo);
        ++k;
      }
      s0 += n[i];
    }
    if (!b2_cat_waves(k, src, start, len, wv + x * 12)) return false;
  }
  return true;
}

}  // namespace lfamd

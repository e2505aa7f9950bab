// Checks sfe::plan_table and sfe::order_norm (scriptrs_amd/csrc/sfe_share.cpp)
// on the host: every frame that the normalisation kernel reads for an item
// must be a raw slot that a log-mel entry writes, with exactly the padded
// samples that the item itself would have used for that frame; the
// reordered normalisation entries are a permutation of the planned ones.
//
// stdin: cases, each "n share" then n lines "start len".  For each case
// prints "case <k> quads <with> <own> tiles <t>" and at the end "bad <count>".
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <tuple>
#include <vector>

#include "sfe_internal.hpp"

using sfe::Item;

// The 512 padded samples of frame f of samples[start, start + len): item
// positions p = 160 f - 256 .. + 511 hold 0 outside [0, len), the sample
// itself at p = 0 (preemphasis restarts there) and x[s] - c x[s - 1] at s =
// start + p elsewhere.  Two frames with equal keys read equal values.
typedef std::tuple<int64_t, int64_t, int64_t, int64_t> Key;
static Key frame_key(int64_t start, int64_t len, int64_t f) {
  const int64_t p0 = sfe::kHop * f - sfe::kPad, p1 = p0 + sfe::kNfft;  // [p0, p1)
  const int64_t lead = p0 < 0 ? std::min<int64_t>(-p0, sfe::kNfft) : 0;
  const int64_t tail = p1 > len ? std::min<int64_t>(p1 - len, sfe::kNfft) : 0;
  const int64_t first = (p0 <= 0 && 0 < p1 && len > 0) ? -p0 : -1;  // index of the restart sample
  // all-zero frames are equal whatever their position
  if (lead + tail >= sfe::kNfft) return Key(0, sfe::kNfft, -1, 0);
  return Key(start + p0, lead, first, tail);
}

int main() {
  int n, share, k = 0;
  long bad = 0;
  while (scanf("%d %d", &n, &share) == 2) {
    std::vector<Item> items(n);
    int64_t fo = 0;
    for (int i = 0; i < n; ++i) {
      long long s, l;
      if (scanf("%lld %lld", &s, &l) != 2) return 2;
      items[i] = sfe::own_item(s, l, 0, sfe::kMel * fo, 0);
      fo += items[i].T;
    }
    sfe::PlanWorkspace ws;
    ws.reserve((size_t)n);
    std::vector<Item> table((size_t)(sfe::kPlanEntriesPerItem + 1) * n);
    size_t n_lm = 0;
    const size_t cap[4] = {ws.sp.capacity(), ws.run_of.capacity(), ws.runs.capacity(), ws.pieces.capacity()};
    const int64_t tiles = sfe::plan_table(items.data(), n, share != 0, &ws, table.data(), &n_lm);
    const size_t cap2[4] = {ws.sp.capacity(), ws.run_of.capacity(), ws.runs.capacity(), ws.pieces.capacity()};
    for (int c = 0; c < 4; ++c)
      if (cap2[c] != cap[c]) {
        printf("case %d: planner list %d grew past reserve(n)\n", k, c);
        ++bad;
      }
    if (n_lm > (size_t)sfe::kPlanEntriesPerItem * n) {
      printf("case %d: %zu log-mel entries for %d items\n", k, n_lm, n);
      ++bad;
    }
    const std::vector<Item> lm(table.begin(), table.begin() + (ptrdiff_t)n_lm);
    const std::vector<Item> norm(table.begin() + (ptrdiff_t)n_lm, table.begin() + (ptrdiff_t)(n_lm + n));
    // order_norm: longest first in classes of 256 frames, output order
    // within one, and the same entries
    std::vector<Item> ordered(norm);
    sfe::order_norm(ordered.data(), n);
    for (int i = 0; i < n; ++i) {
      const Item& a = ordered[i];
      if (i > 0) {
        const Item& p = ordered[i - 1];
        if ((p.T >> 8) < (a.T >> 8) || ((p.T >> 8) == (a.T >> 8) && p.dst_off >= a.dst_off)) {
          printf("case %d: normalisation order broken at %d\n", k, i);
          ++bad;
        }
      }
    }
    {
      // the same entries, byte for byte (dst_off differs between items)
      auto by_dst = [](const Item& a, const Item& b) { return a.dst_off < b.dst_off; };
      std::vector<Item> x(norm), y(ordered);
      std::sort(x.begin(), x.end(), by_dst);
      std::sort(y.begin(), y.end(), by_dst);
      if (memcmp(x.data(), y.data(), x.size() * sizeof(Item)) != 0) {
        printf("case %d: reordered normalisation entries differ\n", k);
        ++bad;
      }
    }
    std::map<int64_t, Key> raw;
    std::map<int64_t, int> members;  // items per shared region
    int64_t quads = 0, own = 0;
    int32_t units = 0;
    for (const Item& e : lm) {
      if (e.unit_off != units || e.n_units < 1) {
        printf("case %d: entry unit_off %d (want %d) n_units %d\n", k, e.unit_off, units, e.n_units);
        ++bad;
      }
      units += e.n_units;
      quads += e.n_units;
      for (int64_t q = e.q0; q < e.q0 + e.n_units; ++q)
        for (int64_t f = 4 * q; f < 4 * q + 4; ++f) {
          const int64_t a = e.out_off + sfe::raw_frame(f);
          if (a < 0 || a >= (int64_t)sfe::kRawTile * tiles) {
            printf("case %d: write outside the scratch at %lld\n", k, (long long)a);
            ++bad;
          }
          if (!raw.emplace(a, frame_key(e.start, e.len, f)).second) {
            printf("case %d: raw slot %lld written twice\n", k, (long long)a);
            ++bad;
          }
        }
    }
    for (int i = 0; i < n; ++i) {
      const Item& it = norm[i];
      own += (items[i].T + 3) / 4;
      if (it.T != items[i].T || it.dst_off != items[i].dst_off) {
        printf("case %d item %d: T or dst_off changed\n", k, i);
        ++bad;
      }
      // the normalisation kernel's 32-bit buffer offsets from the shared
      // region: every load below kNormBufRange bytes
      const int64_t span = std::max(it.out_off, it.tail_off) - it.grid_off + sfe::raw_frame(it.T + 64);
      if (it.out_off < it.grid_off || it.tail_off < it.grid_off ||
          4 * (span + sfe::raw_frame((int64_t)it.gshift + 64)) >= (int64_t)sfe::kNormBufRange) {
        printf("case %d item %d: regions beyond the offsets of the shared region\n", k, i);
        ++bad;
      }
      if (it.f_lo > 0 && ++members[it.grid_off] > sfe::kMaxShareMembers) {
        printf("case %d item %d: more than kMaxShareMembers items share one region\n", k, i);
        ++bad;
      }
      if (it.f_lo > 0 && it.f_hi - it.f_lo + 1 > sfe::kMaxShareFrames) ++bad;
      for (int64_t f = 0; f < it.T; ++f) {
        // the normalisation kernel's address rule
        const bool g = f >= it.f_lo && f <= it.f_hi;
        const int64_t a = (g ? it.grid_off : (f < it.f_lo ? it.out_off : it.tail_off)) +
                          sfe::raw_frame(g ? f + it.gshift : f);
        auto w = raw.find(a);
        if (w == raw.end()) {
          printf("case %d item %d frame %lld: slot %lld never written\n", k, i, (long long)f, (long long)a);
          ++bad;
        } else if (w->second != frame_key(it.start, it.len, f)) {
          printf("case %d item %d frame %lld: slot holds other samples\n", k, i, (long long)f);
          ++bad;
        }
        if (bad > 20) return 1;
      }
    }
    if (!share && quads != own) {
      printf("case %d: sharing off but %lld quads against %lld\n", k, (long long)quads, (long long)own);
      ++bad;
    }
    if (quads > own) {
      printf("case %d: sharing computes more quads (%lld > %lld)\n", k, (long long)quads, (long long)own);
      ++bad;
    }
    printf("case %d quads %lld %lld tiles %lld regions %zu\n", k, (long long)quads, (long long)own, (long long)tiles,
           members.size());
    ++k;
  }
  printf("bad %ld\n", bad);
  return 0;
}

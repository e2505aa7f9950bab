// Log-mel and normalisation tables for a batch of items, with the frames
// that overlapping items share computed once.
//
// The long-form planner (src/long_form/mod.rs, build_fast_execution_plan)
// cuts a recording into chunks that overlap by about 2 s, each featurized
// on its own (src/long_form/worker.rs calls the extractor per chunk).  Every
// chunk starts at a multiple of the hop, so a frame of a later chunk and the
// frame of the earlier chunk centred on the same recording sample read the
// same samples.  The log-mel of such a frame depends only on those samples
// when they lie inside the chunk and after its first sample (preemphasis
// restarts at a chunk's first sample, and zero padding replaces samples
// outside it); frames near a chunk's ends are the chunk's own.  Shared
// frames are bitwise equal to what each chunk would compute: the same
// arithmetic on the same inputs.
//
// Per item of T frames, the interior frames are [2, (len - kPad) / hop]:
// frame f's 512 padded samples (item samples 160 f - 256 .. 160 f + 255)
// then lie in [1, len).  Items whose starts agree modulo the hop and whose
// interior frames overlap or touch form a run; a run's shared log-mel entry
// spans the samples from its first item's start to its last item's end and
// covers the union of their interior frames.  Each item keeps its own first
// quad (frames 0-3) and its last quads (frames past the interior), in tiles
// of its own.  A run is shared only if that computes fewer quads than its
// items would alone.
#include <algorithm>
#include <vector>

#include "sfe_internal.hpp"

namespace sfe {

namespace {

constexpr int kShareLo = 2;        // first interior frame
constexpr int kMinInterior = 32;   // fewer interior frames: the item keeps its own region

struct Span {
  int idx;        // item index
  int64_t res;    // start mod hop
  int64_t c;      // start / hop: the recording frame index of item frame 0
  int64_t lo, hi; // interior frames in recording frame indices
};

int interior_hi(const Item& it) { return (int)((it.len - kPad) / kHop); }

}  // namespace

int64_t plan_items(const Item* items, int n, bool share, std::vector<Item>* lm, std::vector<Item>* norm) {
  lm->clear();
  norm->assign(items, items + n);
  std::vector<int> run_of(n, -1);  // index into runs, or -1: own region
  struct Run {
    int64_t res, lo, hi;  // union of interior frames (recording frame indices)
    int64_t vstart, vend; // samples of the shared entry
    std::vector<int> members;
  };
  std::vector<Run> runs;
  if (share) {
    std::vector<Span> sp;
    for (int i = 0; i < n; ++i) {
      const Item& it = items[i];
      if (it.len < kPad) continue;
      const int hi = interior_hi(it);
      if (hi - kShareLo + 1 < kMinInterior) continue;
      const int64_t c = it.start / kHop;
      sp.push_back({i, it.start % kHop, c, c + kShareLo, c + hi});
    }
    std::sort(sp.begin(), sp.end(), [](const Span& a, const Span& b) {
      return a.res != b.res ? a.res < b.res : (a.lo != b.lo ? a.lo < b.lo : a.idx < b.idx);
    });
    for (size_t k = 0; k < sp.size();) {
      Run r{sp[k].res, sp[k].lo, sp[k].hi, items[sp[k].idx].start, items[sp[k].idx].start + items[sp[k].idx].len, {}};
      r.members.push_back(sp[k].idx);
      size_t m = k + 1;
      // A run's shared frames stay within kMaxShareFrames: the normalisation
      // kernel addresses an item's regions by 32-bit byte offsets from its
      // shared region.
      for (; m < sp.size() && sp[m].res == r.res && sp[m].lo <= r.hi + 1 &&
             std::max(r.hi, sp[m].hi) - r.lo < kMaxShareFrames;
           ++m) {
        const Item& it = items[sp[m].idx];
        r.hi = std::max(r.hi, sp[m].hi);
        r.vstart = std::min(r.vstart, it.start);
        r.vend = std::max(r.vend, it.start + it.len);
        r.members.push_back(sp[m].idx);
      }
      k = m;
      if (r.members.size() < 2) continue;
      // Quads computed with sharing: the run's shared quads plus each item's
      // first and last quads, against each item's own quads.
      const int64_t cv = r.vstart / kHop;
      const int64_t shared = (r.hi - cv) / kQuad - (r.lo - cv) / kQuad + 1;
      int64_t with = shared, without = 0;
      for (int i : r.members) {
        const Item& it = items[i];
        const int64_t nq = (it.T + kQuad - 1) / kQuad;
        const int64_t qa = (interior_hi(it) + 1) / kQuad;
        with += 1 + (nq - qa);
        without += nq;
      }
      if (with >= without) continue;
      for (int i : r.members) run_of[i] = (int)runs.size();
      runs.push_back(std::move(r));
    }
  }

  // Raw regions, in item order (a run's shared region and its members' own
  // tiles where its first member is), and log-mel entries.  The shared
  // entry is cut at its members' starts, and all entries are then ordered by
  // the recording position of their first frame: the first and last quads
  // of items, whose samples cross an item's ends and take the kernel's
  // slower per-sample path, are spread over the launch instead of falling
  // to a few waves.
  int64_t tiles = 0;
  std::vector<std::pair<int64_t, Item>> pieces;  // (position, entry)
  std::vector<int64_t> run_grid(runs.size(), -1);  // grid_off of each run
  std::vector<int64_t> run_cv(runs.size(), 0);
  auto add_entry = [&](int64_t start, int64_t len, int q0, int q1, int64_t region) -> Item {
    // quads [q0, q1] of the samples [start, start + len), written to tiles
    // from `region` on
    Item e{};
    e.start = start;
    e.len = len;
    e.T = (int32_t)(len / kHop + 1);
    e.q0 = q0;
    e.n_units = q1 - q0 + 1;
    e.out_off = region - (int64_t)kRawTile * (q0 / 4);
    e.grid_off = e.out_off;
    e.tail_off = e.out_off;
    e.f_lo = 0;
    e.f_hi = e.T - 1;
    tiles += (int64_t)q1 / 4 - q0 / 4 + 1;
    return e;
  };
  auto add_piece = [&](const Item& e, int q0, int q1) {
    Item p = e;
    p.q0 = q0;
    p.n_units = q1 - q0 + 1;
    pieces.emplace_back(e.start + (int64_t)kHop * kQuad * q0, p);
  };
  for (int i = 0; i < n; ++i) {
    const Item& it = items[i];
    Item& nt = (*norm)[i];
    const int nq = (it.T + kQuad - 1) / kQuad;
    const int r = run_of[i];
    if (r < 0) {
      const Item e = add_entry(it.start, it.len, 0, nq - 1, (int64_t)kRawTile * tiles);
      add_piece(e, 0, nq - 1);
      nt.out_off = nt.grid_off = nt.tail_off = e.out_off;
      nt.f_lo = 0;
      nt.f_hi = it.T - 1;
      nt.gshift = 0;
      continue;
    }
    const Run& run = runs[r];
    if (run_grid[r] < 0) {
      // The run's shared region, then its members' own first and last
      // tiles, all at once: the members' regions follow the shared one
      // closely (the normalisation kernel's 32-bit offsets).
      const int64_t cv = run.vstart / kHop;
      const int q_lo = (int)((run.lo - cv) / kQuad), q_hi = (int)((run.hi - cv) / kQuad);
      const Item e = add_entry(run.vstart, run.vend - run.vstart, q_lo, q_hi, (int64_t)kRawTile * tiles);
      run_cv[r] = cv;
      run_grid[r] = e.out_off;
      // cut points: the quads where members start
      std::vector<int> cuts;
      for (int m : run.members) {
        const int q = (int)((items[m].start / kHop - cv) / kQuad);
        if (q > q_lo && q <= q_hi) cuts.push_back(q);
      }
      std::sort(cuts.begin(), cuts.end());
      cuts.erase(std::unique(cuts.begin(), cuts.end()), cuts.end());
      int q = q_lo;
      for (int c : cuts) {
        add_piece(e, q, c - 1);
        q = c;
      }
      add_piece(e, q, q_hi);
      for (int m : run.members) {
        const Item& mt = items[m];
        const int mq = (mt.T + kQuad - 1) / kQuad;
        const int qa = (interior_hi(mt) + 1) / kQuad;
        const Item head = add_entry(mt.start, mt.len, 0, 0, (int64_t)kRawTile * tiles);
        add_piece(head, 0, 0);
        const Item tail = add_entry(mt.start, mt.len, qa, mq - 1, (int64_t)kRawTile * tiles);
        add_piece(tail, qa, mq - 1);
        Item& nm = (*norm)[m];
        nm.out_off = head.out_off;
        nm.tail_off = tail.out_off;
        nm.grid_off = run_grid[r];
        nm.f_lo = kShareLo;
        nm.f_hi = interior_hi(mt);
        nm.gshift = (int32_t)(mt.start / kHop - cv);
      }
    }
  }
  // Stable: pieces at one position keep their order of creation (an item's
  // own quads are one piece, so it stays whole).
  std::stable_sort(pieces.begin(), pieces.end(),
                   [](const std::pair<int64_t, Item>& a, const std::pair<int64_t, Item>& b) { return a.first < b.first; });
  int32_t units = 0;
  for (auto& pc : pieces) {
    pc.second.unit_off = units;
    units += pc.second.n_units;
    lm->push_back(pc.second);
  }
  for (Item& nt : *norm) {
    nt.unit_off = 0;
    nt.n_units = 0;
    nt.q0 = 0;
  }
  return tiles;
}

}  // namespace sfe

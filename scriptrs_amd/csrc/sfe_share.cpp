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

constexpr int kShareLo = 2;       // first interior frame
constexpr int kMinInterior = 32;  // fewer interior frames: the item keeps its own region

int interior_hi(const Item& it) { return (int)((it.len - kPad) / kHop); }

}  // namespace

void PlanWorkspace::reserve(size_t n) {
  sp.reserve(n);
  run_of.reserve(n);
  runs.reserve(n);
  pieces.reserve((size_t)kPlanEntriesPerItem * n);
}

int64_t plan_table(const Item* items, int n, bool share, PlanWorkspace* ws, Item* table, size_t* n_lm) {
  // (every container below stays within the capacity reserve(n) gave it)
  Item* norm = table + (size_t)kPlanEntriesPerItem * n;  // staged here, moved down at the end
  for (int i = 0; i < n; ++i) norm[i] = items[i];
  std::vector<int>& run_of = ws->run_of;
  run_of.assign(n, -1);  // index into runs, or -1: own region
  std::vector<PlanWorkspace::Run>& runs = ws->runs;
  runs.clear();
  if (share) {
    std::vector<PlanWorkspace::Span>& sp = ws->sp;
    sp.clear();
    for (int i = 0; i < n; ++i) {
      const Item& it = items[i];
      if (it.len < kPad) continue;
      const int hi = interior_hi(it);
      if (hi - kShareLo + 1 < kMinInterior) continue;
      const int64_t c = it.start / kHop;
      sp.push_back({i, it.start % kHop, c + kShareLo, c + hi});
    }
    std::sort(sp.begin(), sp.end(), [](const PlanWorkspace::Span& a, const PlanWorkspace::Span& b) {
      return a.res != b.res ? a.res < b.res : (a.lo != b.lo ? a.lo < b.lo : a.idx < b.idx);
    });
    for (size_t k = 0; k < sp.size();) {
      const Item& f = items[sp[k].idx];
      PlanWorkspace::Run r{sp[k].res, sp[k].lo, sp[k].hi, f.start, f.start + f.len, 0, -1, (int)k, (int)k + 1};
      // A run's shared frames and members stay within kMaxShareFrames and
      // kMaxShareMembers: the normalisation kernel addresses an item's
      // regions by 32-bit byte offsets from its shared region.
      for (size_t m = k + 1; m < sp.size() && sp[m].res == r.res && sp[m].lo <= r.hi + 1 &&
                             std::max(r.hi, sp[m].hi) - r.lo < kMaxShareFrames && (int)m - r.k0 < kMaxShareMembers;
           ++m) {
        const Item& it = items[sp[m].idx];
        r.hi = std::max(r.hi, sp[m].hi);
        r.vstart = std::min(r.vstart, it.start);
        r.vend = std::max(r.vend, it.start + it.len);
        r.k1 = (int)m + 1;
      }
      k = (size_t)r.k1;
      if (r.k1 - r.k0 < 2) continue;
      // Quads computed with sharing: the run's shared quads plus each item's
      // first and last quads, against each item's own quads.
      r.cv = r.vstart / kHop;
      const int64_t shared = (r.hi - r.cv) / kQuad - (r.lo - r.cv) / kQuad + 1;
      int64_t with = shared, without = 0;
      for (int j = r.k0; j < r.k1; ++j) {
        const Item& it = items[sp[j].idx];
        const int64_t nq = (it.T + kQuad - 1) / kQuad;
        const int64_t qa = (interior_hi(it) + 1) / kQuad;
        with += 1 + (nq - qa);
        without += nq;
      }
      if (with >= without) continue;
      for (int j = r.k0; j < r.k1; ++j) run_of[sp[j].idx] = (int)runs.size();
      runs.push_back(r);
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
  std::vector<PlanWorkspace::Piece>& pieces = ws->pieces;
  pieces.clear();
  auto add_entry = [&](int64_t start, int64_t len, int q0, int q1) -> Item {
    // quads [q0, q1] of the samples [start, start + len), written to the
    // next free tiles
    Item e{};
    e.start = start;
    e.len = len;
    e.T = (int32_t)(len / kHop + 1);
    e.q0 = q0;
    e.n_units = q1 - q0 + 1;
    e.out_off = (int64_t)kRawTile * (tiles - q0 / 4);
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
    pieces.push_back({e.start + (int64_t)kHop * kQuad * q0, (int32_t)pieces.size(), p});
  };
  for (int i = 0; i < n; ++i) {
    const Item& it = items[i];
    const int r = run_of[i];
    if (r < 0) {
      const int nq = (it.T + kQuad - 1) / kQuad;
      const Item e = add_entry(it.start, it.len, 0, nq - 1);
      add_piece(e, 0, nq - 1);
      Item& nt = norm[i];
      nt.out_off = nt.grid_off = nt.tail_off = e.out_off;
      nt.f_lo = 0;
      nt.f_hi = it.T - 1;
      nt.gshift = 0;
      continue;
    }
    PlanWorkspace::Run& run = runs[r];
    if (run.grid >= 0) continue;  // planned with its first member
    // The run's shared region, then its members' own first and last tiles,
    // all at once: the members' regions follow the shared one closely (the
    // normalisation kernel's 32-bit offsets).
    const int64_t cv = run.cv;
    const int q_lo = (int)((run.lo - cv) / kQuad), q_hi = (int)((run.hi - cv) / kQuad);
    const Item e = add_entry(run.vstart, run.vend - run.vstart, q_lo, q_hi);
    run.grid = e.out_off;
    // cut at the quads where members start (members are in start order)
    int q = q_lo;
    for (int j = run.k0; j < run.k1; ++j) {
      const int c = (int)((items[ws->sp[j].idx].start / kHop - cv) / kQuad);
      if (c > q && c <= q_hi) {
        add_piece(e, q, c - 1);
        q = c;
      }
    }
    add_piece(e, q, q_hi);
    for (int j = run.k0; j < run.k1; ++j) {
      const int m = ws->sp[j].idx;
      const Item& mt = items[m];
      const int mq = (mt.T + kQuad - 1) / kQuad;
      const int qa = (interior_hi(mt) + 1) / kQuad;
      const Item head = add_entry(mt.start, mt.len, 0, 0);
      add_piece(head, 0, 0);
      const Item tail = add_entry(mt.start, mt.len, qa, mq - 1);
      add_piece(tail, qa, mq - 1);
      Item& nm = norm[m];
      nm.out_off = head.out_off;
      nm.tail_off = tail.out_off;
      nm.grid_off = run.grid;
      nm.f_lo = kShareLo;
      nm.f_hi = interior_hi(mt);
      nm.gshift = (int32_t)(mt.start / kHop - cv);
    }
  }
  // By position; pieces at one position keep their order of creation (an
  // item's own quads are one piece, so it stays whole).
  std::sort(pieces.begin(), pieces.end(), [](const PlanWorkspace::Piece& a, const PlanWorkspace::Piece& b) {
    return a.pos != b.pos ? a.pos < b.pos : a.seq < b.seq;
  });
  int32_t units = 0;
  for (size_t k = 0; k < pieces.size(); ++k) {
    table[k] = pieces[k].e;
    table[k].unit_off = units;
    units += pieces[k].e.n_units;
  }
  *n_lm = pieces.size();
  for (int i = 0; i < n; ++i) {
    Item nt = norm[i];
    nt.unit_off = 0;
    nt.n_units = 0;
    nt.q0 = 0;
    table[*n_lm + i] = nt;
  }
  return tiles;
}

void order_norm(Item* norm, int n) {
  // Normalisation workgroups start in table order: longest items first (in
  // classes of 256 frames, call order within one), so the last ones to start
  // are short; each entry writes its own dst_off, which rises with the call
  // order.  Ragged batches (config 4): 0.0738 -> 0.0712 ms.
  std::sort(norm, norm + n, [](const Item& a, const Item& b) {
    return (a.T >> 8) != (b.T >> 8) ? (a.T >> 8) > (b.T >> 8) : a.dst_off < b.dst_off;
  });
}

}  // namespace sfe

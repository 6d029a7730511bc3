// Host side of the workgroup dispatch order (the header states the scheme).
#include "dispatch_order.h"

#include <stdlib.h>

#include <algorithm>
#include <map>
#include <memory>
#include <mutex>
#include <set>
#include <tuple>
#include <utility>
#include <vector>

namespace mm1 {
namespace {

// Modelled cost of one row block: its 64-key tiles plus the fixed cost of a
// workgroup (operand loads, ring fill, stores), in units of one key tile.
constexpr int kRowBlockFixed = 1;

std::vector<int> item_costs(const GridShape& g) {
  const int G = g.H / g.Hkv, R = G * g.S, nbg = g.B * g.Hkv;
  const int n_tiles = (R + g.rows - 1) / g.rows;
  std::vector<int> cost((size_t)n_tiles * nbg);
  for (size_t j = 0; j < cost.size(); ++j) {
    const int tile = n_tiles - 1 - (int)(j / nbg);
    const int last_row = std::min(tile * g.rows + g.rows, R) - 1;
    cost[j] = std::min(g.S - 1, last_row / G) / 64 + 1 + kRowBlockFixed;
  }
  return cost;
}

// Order in which one CU group (a shader engine: `slots` workgroup slots)
// should receive `cost`'s items: pack them into bins of near-equal cost (the
// largest remaining item, then the largest ones that still fit under the
// target; the target grows until every item is placed), then list the items
// by the modelled time at which their bin's slot asks for them.
std::vector<int> lane_order(const std::vector<int>& cost, int slots) {
  const int n = (int)cost.size();
  long total = 0;
  int largest = 0;
  for (int c : cost) {
    total += c;
    largest = std::max(largest, c);
  }
  std::vector<std::vector<int>> bins;
  bool packed = false;
  long target = std::max<long>((total + slots - 1) / slots, largest);
  for (int tries = 0; tries < 4096 && !packed; ++tries) {
    std::multiset<std::pair<int, int>> rem;
    for (int i = 0; i < n; ++i) rem.emplace(cost[i], i);
    bins.assign(slots, {});
    for (int b = 0; b < slots && !rem.empty(); ++b) {
      auto top = std::prev(rem.end());
      long load = top->first;
      bins[b].push_back(top->second);
      rem.erase(top);
      while (!rem.empty()) {
        auto it = rem.upper_bound({(int)std::min<long>(target - load, 1 << 30), 1 << 30});
        if (it == rem.begin()) break;
        --it;
        load += it->first;
        bins[b].push_back(it->second);
        rem.erase(it);
      }
    }
    packed = rem.empty();
    target += std::max<long>(1, target >> 6);
  }
  std::vector<int> order;
  if (!packed) {   // not reached for the grids here; longest first
    order.resize(n);
    for (int i = 0; i < n; ++i) order[i] = i;
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return cost[a] > cost[b]; });
    return order;
  }
  std::vector<std::tuple<long, int, int>> ev;   // (time the slot asks, bin, item)
  for (int b = 0; b < slots; ++b) {
    long t = 0;
    for (int i : bins[b]) {
      ev.emplace_back(t, b, i);
      t += cost[i];
    }
  }
  std::sort(ev.begin(), ev.end());
  order.reserve(n);
  for (const auto& e : ev) order.push_back(std::get<2>(e));
  return order;
}

constexpr int kSe = 4;   // shader engines per XCD

// Modelled end time of one XCD's stream (-1: no item): the k-th workgroup
// goes to SE k % kSe and waits, in order, for the first free of that SE's
// `slots_per_se` slots.
long stream_span(const std::vector<int>& stream, const std::vector<int>& cost, int slots_per_se) {
  std::vector<std::multiset<long>> free(kSe);
  for (auto& f : free)
    for (int i = 0; i < slots_per_se; ++i) f.insert(0);
  long last = 0, end = 0;
  for (size_t k = 0; k < stream.size(); ++k) {
    auto& f = free[k % kSe];
    const long t = std::max(*f.begin(), last);
    f.erase(f.begin());
    last = t;
    const long e = t + (stream[k] < 0 ? 0 : cost[stream[k]]);
    f.insert(e);
    end = std::max(end, e);
  }
  return end;
}

// An XCD hands its k-th workgroup to shader engine k % 4 (a fixed
// permutation of its 4 SEs, each with a quarter of the XCD's CUs) and waits,
// in order, until that SE has a free slot.  Candidate streams: deal the
// XCD's items to 4 lanes, longest first in a snake (each lane gets the same
// mix of sizes), order each lane longest first or packed for its SE's slots,
// and interleave the lanes position by position so that the 4 SEs ask for
// their j-th item at about the same time.  Returns the stream (-1: no item).
std::vector<int> snake_stream(const std::vector<int>& cost, int slots_per_se, bool pack) {
  const int n = (int)cost.size();
  std::vector<int> srt(n);
  for (int i = 0; i < n; ++i) srt[i] = i;
  std::stable_sort(srt.begin(), srt.end(), [&](int a, int b) { return cost[a] > cost[b]; });
  std::vector<std::vector<int>> lanes(kSe);
  for (int r = 0; r < n; ++r) {
    const int blk = r / kSe, k = r % kSe;
    lanes[blk % 2 == 0 ? k : kSe - 1 - k].push_back(srt[r]);
  }
  size_t longest = 0;
  for (auto& ln : lanes) {
    if (pack) {
      std::vector<int> c;
      for (int i : ln) c.push_back(cost[i]);
      const std::vector<int> ord = lane_order(c, slots_per_se);
      std::vector<int> seq;
      for (int j : ord) seq.push_back(ln[j]);
      ln.swap(seq);
    }
    longest = std::max(longest, ln.size());
  }
  std::vector<int> stream;
  for (size_t j = 0; j < longest; ++j)
    for (int k = 0; k < kSe; ++k) stream.push_back(j < lanes[k].size() ? lanes[k][j] : -1);
  while (!stream.empty() && stream.back() < 0) stream.pop_back();
  return stream;
}

// Builds the table for items with the given modelled costs (-1: an empty
// item, which runs in no slot of a table), `slots_per_se` workgroup slots per
// shader engine.  Per XCD it keeps the best-rated of the default order and
// the two snake streams.  Returns the modelled span of the order kept
// (out.n == 0: the default order, whose slots include the empty items).
long build_from_costs(const std::vector<int>& cost_in, int slots_per_se, DispatchOrder& out) {
  out.n = 0;
  const int n = (int)cost_in.size();
  if (n == 0) return 0;
  std::vector<std::vector<int>> streams(8);
  size_t rounds = 0;
  bool any_change = false;
  long span_default = 0, span_best = 0;
  for (int x = 0; x < 8; ++x) {
    // this XCD's items (default numbering) and their costs; the default
    // stream also keeps its empty slots
    std::vector<int> mine, c, dflt;
    for (int j = x; j < n; j += 8) {
      if (cost_in[j] >= 0) {
        dflt.push_back((int)mine.size());
        mine.push_back(j);
        c.push_back(cost_in[j]);
      } else {
        dflt.push_back(-1);
      }
    }
    std::vector<int> best = dflt;
    long best_span = stream_span(best, c, slots_per_se);
    span_default = std::max(span_default, best_span);
    for (bool pack : {false, true}) {
      if (c.empty()) break;
      std::vector<int> cand = snake_stream(c, slots_per_se, pack);
      const long span = stream_span(cand, c, slots_per_se);
      if (span < best_span) {
        best_span = span;
        best.swap(cand);
        any_change = true;
      }
    }
    span_best = std::max(span_best, best_span);
    for (int i : best) streams[x].push_back(i < 0 ? -1 : mine[i]);
    rounds = std::max(rounds, streams[x].size());
  }
  if (!any_change || 8 * rounds > (size_t)kOrderCap || n > (int)kNoItem) return span_default;
  for (int i = 0; i < kOrderCap; ++i) out.item[i] = kNoItem;
  for (int x = 0; x < 8; ++x)
    for (size_t r = 0; r < streams[x].size(); ++r)
      if (streams[x][r] >= 0) out.item[8 * r + x] = (uint16_t)streams[x][r];
  out.n = (int)(8 * rounds);
  return span_best;
}

void build(const GridShape& g, int cus, DispatchOrder& out) {
  const int slots_per_se = std::max(1, cus / (8 * kSe)) * std::max(1, g.wg_per_cu);
  build_from_costs(item_costs(g), slots_per_se, out);
}

// Grouped dK/dV: modelled cost of a chunk, in 32-query tiles: its tiles, the
// fixed cost of a workgroup (K/V loads, ring fill, pipeline drain, stores)
// and, for a chunk of a split key tile, its fp32 partial stores and their
// share of the reduction.
constexpr int kDkdvFixed = 6;
constexpr int kDkdvSplit = 2;

std::vector<int> dkdv_costs(int B, int S, int G, int Hkv, bool causal, int L, int C) {
  const int n_kt = (S + 127) / 128, nbg = B * Hkv;
  std::vector<int> cost((size_t)n_kt * C * nbg, -1);
  for (int kt = 0; kt < n_kt; ++kt) {
    const int len = G * dkdv_n_qt(S, kt, causal);
    const int nc = dkdv_chunks(len, L, C);
    for (int c = 0; c < nc; ++c) {
      const int size = (len - c + nc - 1) / nc;
      const int cc = size + kDkdvFixed + (nc > 1 ? kDkdvSplit : 0);
      for (int bg = 0; bg < nbg; ++bg) cost[((size_t)kt * C + c) * nbg + bg] = cc;
    }
  }
  return cost;
}

// Chunk length: the candidate (fractions of the per-CU share of the work,
// and no split at all) whose order the dispatch model rates fastest; on a
// tie the one with fewer split key tiles.
void build_dkdv(int B, int S, int H, int Hkv, bool causal, int cus, DkdvPlan& plan) {
  const int G = H / Hkv, n_kt = (S + 127) / 128, nbg = B * Hkv;
  const int C = G;
  long total = 0;
  int longest = 0;
  for (int kt = 0; kt < n_kt; ++kt) {
    const int len = G * dkdv_n_qt(S, kt, causal);
    total += (long)len * nbg;
    longest = std::max(longest, len);
  }
  const long share = std::max<long>(1, (total + cus - 1) / std::max(1, cus));
  const int slots_per_se = std::max(1, cus / (8 * kSe));
  std::vector<long> cands = {share / 3, share / 2, (2 * share) / 3, share, (4 * share) / 3, longest};
  long best_span = -1;
  plan.C = C;
  for (long cand : cands) {
    const int L = (int)std::min<long>(std::max<long>(1, cand), longest);
    auto ord = std::make_unique<DispatchOrder>();
    const long span = build_from_costs(dkdv_costs(B, S, G, Hkv, causal, L, C), slots_per_se, *ord);
    if (best_span < 0 || span < best_span || (span == best_span && L > plan.L)) {
      best_span = span;
      plan.L = L;
      plan.order = *ord;
    }
  }
  plan.n_items = n_kt * C * nbg;
  plan.split_keys = 0;
  for (int kt = 0; kt < n_kt; ++kt)
    if (dkdv_chunks(G * dkdv_n_qt(S, kt, causal), plan.L, C) > 1)
      plan.split_keys = std::min(S, 128 * (kt + 1));
}

bool order_enabled() {
  const char* e = getenv("MM1_DISPATCH_ORDER");
  return !(e && e[0] == '0');
}

int device_cus() {
  static int cached[64];
  static std::once_flag once[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::call_once(once[dev], [dev] {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
    cached[dev] = cus;
  });
  return cached[dev];
}

const DispatchOrder& default_order() {
  static const DispatchOrder d = [] {
    DispatchOrder o;
    o.n = 0;
    for (int i = 0; i < kOrderCap; ++i) o.item[i] = kNoItem;
    return o;
  }();
  return d;
}

}  // namespace

GridShape row_block_grid(int variant, int B, int S, int H, int Hkv) {
  return {B, S, H, Hkv, variant == 1 ? 128 : 256, variant == 1 ? 2 : 1};
}

GridShape dq_grid(int variant, int B, int S, int H, int Hkv) {
  return {B, S, H, Hkv, variant == 0 ? 128 : 256, variant == 0 ? 2 : 1};
}

const DispatchOrder& dispatch_order_for(const GridShape& g, bool causal, int cus) {
  if (!causal || !order_enabled() || cus <= 0 || g.wg_per_cu != 1) return default_order();
  using Key = std::tuple<int, int, int, int, int, int>;
  static std::mutex mu;
  static std::map<Key, std::unique_ptr<DispatchOrder>> cache;
  const Key key{g.B, g.S, g.H, g.Hkv, g.rows, cus};
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find(key);
  if (it == cache.end()) {
    auto ord = std::make_unique<DispatchOrder>();
    build(g, cus, *ord);
    it = cache.emplace(key, std::move(ord)).first;
  }
  return it->second->n ? *it->second : default_order();
}

const DispatchOrder& dispatch_order(const GridShape& g, bool causal) {
  if (!causal || !order_enabled()) return default_order();
  return dispatch_order_for(g, causal, device_cus());
}

const DkdvPlan& dkdv_plan_for(int B, int S, int H, int Hkv, bool causal, int cus) {
  // The chunk length (and so the partial-sum layout) depends on the shape and
  // the CU count only; the dispatch-order switch changes which launch slot
  // runs which item, not the items.
  const bool ordered = order_enabled();
  using Key = std::tuple<int, int, int, int, bool, int, bool>;
  const Key key{B, S, H, Hkv, causal, cus, ordered};
  static std::mutex mu;
  static std::map<Key, std::unique_ptr<DkdvPlan>> cache;
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find(key);
  if (it == cache.end()) {
    auto plan = std::make_unique<DkdvPlan>();
    build_dkdv(B, S, H, Hkv, causal, std::max(1, cus), *plan);
    if (!ordered) plan->order.n = 0;
    it = cache.emplace(key, std::move(plan)).first;
  }
  return *it->second;
}

const DkdvPlan& dkdv_plan(int B, int S, int H, int Hkv, bool causal) {
  return dkdv_plan_for(B, S, H, Hkv, causal, device_cus());
}

}  // namespace mm1

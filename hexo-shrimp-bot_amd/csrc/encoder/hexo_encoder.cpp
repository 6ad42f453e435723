// Native Hexo rules subset + MantisNet position encoder (host C++).
//
// What it restates (reference file:line):
//   rules: legal frontier in canonical (q, r) order, turn pattern, six-in-a-row
//          (crates/hexo-engine/README.md:47-50, 111-115, 197-200;
//           crates/hexo-engine/src/position.rs:384-389)
//   encoder::build            crates/models/mantisnet/src/encoder.rs:1047-1355
//   encoder::cell_node_fields encoder.rs:943-1039
//   encoder::collate          encoder.rs:1512-1625 (+ collate_action_fields :1431-1510)
//   relay_tables              python/mantisnet/mantisnet/relay.py:48-94
//
// Design: every position is encoded on a dense local grid (stone index,
// legal index and window-start planes over the stone bounding box plus the
// 14-cell reach of a window through a legal cell), so every lookup is one
// array read and every ordering the representation fixes — windows by
// (q*2^21 + r)*4 + axis, radius edges destination-major / source-ascending,
// adjacency by (dst, src, axis) — falls out of a row-major scan with no sort.
// Positions build in parallel; collation fills disjoint slices in parallel.
#include "../../../include/hexo_encoder.h"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <array>
#include <atomic>
#include <cstdio>
#include <cstring>
#include <set>
#include <stdexcept>
#include <string>
#include <thread>
#include <tuple>
#include <vector>

namespace {

constexpr int kWin = 6;
constexpr int kRadius = 8;
constexpr int kTactical = 11;
// vocabulary sizes (encoder.rs:127-137, :274): window ranks, occupancy,
// decoder and post-placement classes
constexpr int64_t kTernPatterns = 377, kTernOcc = 1458, kTernDec = 726, kTernPost1 = 729;
constexpr int kThreatCap = 8;
constexpr int kDecClasses = 726;
constexpr int kGlobalRows = 4;
constexpr int kCoordLimit = 16000;
constexpr int AQ[3] = {1, 0, 1};
constexpr int AR[3] = {0, 1, -1};

struct Failure : std::runtime_error {
  int code;
  Failure(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

[[noreturn]] void fail(int code, const std::string& msg) { throw Failure(code, msg); }

inline int hexdist(int dq, int dr) {
  return std::max({std::abs(dq), std::abs(dr), std::abs(dq + dr)});
}

// ------------------------------------------------------------- vocabularies

struct Vocab {
  int pow3[kWin];
  int rev[729];
  int rank[729];
  int dec[729][kWin];
  int occ[729][kWin];
  int post1[729][kWin];
  int orbit[25][25];
  int empty_cls[3];
  std::vector<float> counts;  // (377, 1458)

  int digit(int p, int s) const { return p / pow3[s] % 3; }

  Vocab() {
    pow3[0] = 1;
    for (int s = 1; s < kWin; ++s) pow3[s] = pow3[s - 1] * 3;
    for (int p = 0; p < 729; ++p) {
      int r = 0;
      for (int s = 0; s < kWin; ++s) r = r * 3 + digit(p, s);
      rev[p] = r;
    }
    // Reversal-canonical pattern ranks over the nonempty patterns.
    std::vector<int> canon;
    for (int p = 1; p < 729; ++p) canon.push_back(std::min(p, rev[p]));
    std::sort(canon.begin(), canon.end());
    canon.erase(std::unique(canon.begin(), canon.end()), canon.end());
    if (canon.size() != 377) fail(HEXO_E_INTERNAL, "pattern vocabulary is not 377");
    rank[0] = -1;
    for (int p = 1; p < 729; ++p)
      rank[p] = int(std::lower_bound(canon.begin(), canon.end(), std::min(p, rev[p])) -
                    canon.begin());
    // Joint (pattern, slot) orbits of (p, s) -> (rev p, 5 - s); the orbit id
    // is the first member in ascending (p, s) order.
    static int joint[729][kWin];
    int nxt = 0;
    for (int p = 0; p < 729; ++p)
      for (int s = 0; s < kWin; ++s) {
        int rp = rev[p], rs = kWin - 1 - s;
        joint[p][s] = std::make_pair(p, s) <= std::make_pair(rp, rs) ? nxt++ : joint[rp][rs];
      }
    if (nxt != 2187) fail(HEXO_E_INTERNAL, "joint orbit count is not 2187");
    auto restrict_rank = [&](auto in_set, int (*out)[kWin], int expect) {
      std::vector<int> ids;
      for (int p = 0; p < 729; ++p)
        for (int s = 0; s < kWin; ++s)
          if (in_set(p, s)) ids.push_back(joint[p][s]);
      std::sort(ids.begin(), ids.end());
      ids.erase(std::unique(ids.begin(), ids.end()), ids.end());
      if (int(ids.size()) != expect) fail(HEXO_E_INTERNAL, "class vocabulary size");
      for (int p = 0; p < 729; ++p)
        for (int s = 0; s < kWin; ++s)
          out[p][s] = in_set(p, s)
                          ? int(std::lower_bound(ids.begin(), ids.end(), joint[p][s]) - ids.begin())
                          : -1;
    };
    restrict_rank([&](int p, int s) { return p != 0 && digit(p, s) == 0; }, dec, 726);
    restrict_rank([&](int p, int s) { return digit(p, s) != 0; }, occ, 1458);
    // Post-placement orbits over own-digit slots.
    nxt = 0;
    for (int p = 0; p < 729; ++p)
      for (int s = 0; s < kWin; ++s) {
        if (digit(p, s) != 1) {
          post1[p][s] = -1;
          continue;
        }
        int rp = rev[p], rs = kWin - 1 - s;
        post1[p][s] = std::make_pair(p, s) <= std::make_pair(rp, rs) ? nxt++ : post1[rp][rs];
      }
    if (nxt != 729) fail(HEXO_E_INTERNAL, "post-placement vocabulary is not 729");
    for (int k = 0; k < 3; ++k) empty_cls[k] = post1[pow3[k]][k];
    // D6 displacement orbits within radius 12, ranked by (distance, canonical).
    auto canonical = [](int q, int r) {
      std::pair<int, int> best{q, r};
      for (int refl = 0; refl < 2; ++refl) {
        int iq = refl ? r : q, ir = refl ? q : r;
        for (int k = 0; k < 6; ++k) {
          best = std::min(best, std::make_pair(iq, ir));
          int nq = -ir, nr = iq + ir;
          iq = nq;
          ir = nr;
        }
      }
      return best;
    };
    std::set<std::tuple<int, int, int>> reps;
    for (int q = -12; q <= 12; ++q)
      for (int r = -12; r <= 12; ++r) {
        int d = hexdist(q, r);
        if (d >= 1 && d <= 12) {
          auto c = canonical(q, r);
          reps.insert({d, c.first, c.second});
        }
      }
    if (reps.size() != 48) fail(HEXO_E_INTERNAL, "orbit vocabulary is not 48");
    std::vector<std::tuple<int, int, int>> sorted(reps.begin(), reps.end());
    for (int q = -12; q <= 12; ++q)
      for (int r = -12; r <= 12; ++r) {
        int d = hexdist(q, r);
        orbit[q + 12][r + 12] = -1;
        if (d < 1 || d > 12) continue;
        auto c = canonical(q, r);
        orbit[q + 12][r + 12] = int(
            std::lower_bound(sorted.begin(), sorted.end(), std::make_tuple(d, c.first, c.second)) -
            sorted.begin());
      }
    counts.assign(size_t(377) * 1458, 0.f);
    for (int p = 1; p < 729; ++p) {
      if (p > rev[p]) continue;  // one representative per reversal orbit
      for (int s = 0; s < kWin; ++s)
        if (occ[p][s] >= 0) counts[size_t(rank[p]) * 1458 + occ[p][s]] += 1.f;
    }
  }
};

const Vocab& vocab() {
  static const Vocab v;
  return v;
}

// ------------------------------------------------------------- local grid

template <typename T>
struct Grid {
  int q0 = 0, r0 = 0, nq = 0, nr = 0;
  std::vector<T> v;
  void init(int qlo, int qhi, int rlo, int rhi, T fill) {
    q0 = qlo;
    r0 = rlo;
    nq = qhi - qlo + 1;
    nr = rhi - rlo + 1;
    if (size_t(nq) * size_t(nr) > (size_t(1) << 26)) fail(HEXO_E_LIMIT, "board extent too large");
    v.assign(size_t(nq) * size_t(nr), fill);
  }
  bool inside(int q, int r) const {
    return q >= q0 && r >= r0 && q < q0 + nq && r < r0 + nr;
  }
  T& at(int q, int r) { return v[size_t(q - q0) * nr + (r - r0)]; }
  T get(int q, int r, T dflt) const {
    return inside(q, r) ? v[size_t(q - q0) * nr + (r - r0)] : dflt;
  }
};

// ------------------------------------------------------------- rules

struct Position {
  std::vector<std::array<int, 3>> stones;  // (q, r, owner), canonical (q, r) order
  std::vector<std::array<int, 2>> legal;   // canonical order
  int mover = 0;
  int moves_remaining = 1;
  int winner = -1;  // set when the last placement completed six (terminal replays only)
};

inline int mover_after(int64_t ply) { return ply == 0 ? 0 : (((ply - 1) / 2) % 2 == 0 ? 1 : 0); }
inline int remaining_after(int64_t ply) { return ply == 0 ? 1 : (ply % 2 == 1 ? 2 : 1); }

// Six or more of `who` in a row through (q, r) if `who` stood there.
bool completes_six(const Grid<int8_t>& owner, int q, int r, int who) {
  for (int a = 0; a < 3; ++a) {
    int run = 1;
    for (int sign = -1; sign <= 1; sign += 2)
      for (int k = 1; k < kWin; ++k) {
        if (owner.get(q + sign * k * AQ[a], r + sign * k * AR[a], -1) != who) break;
        ++run;
      }
    if (run >= kWin) return true;
  }
  return false;
}

// Replay a placement sequence through the rules and return the position.
// A sequence whose last placement completes six is refused unless
// allow_terminal: then the position is terminal (no legal placements, the
// winner to move, as the engine freezes it).
Position replay(const int16_t* moves, int64_t n, bool allow_terminal = false) {
  Position pos;
  int qlo = 0, qhi = 0, rlo = 0, rhi = 0;
  for (int64_t i = 0; i < n; ++i) {
    int q = moves[2 * i], r = moves[2 * i + 1];
    if (std::abs(q) > kCoordLimit || std::abs(r) > kCoordLimit || std::abs(q + r) > kCoordLimit)
      fail(HEXO_E_LIMIT, "placement outside the coordinate domain");
    qlo = std::min(qlo, q), qhi = std::max(qhi, q), rlo = std::min(rlo, r), rhi = std::max(rhi, r);
  }
  const int m = kRadius + 1;
  Grid<int8_t> owner, cover;
  owner.init(qlo - m, qhi + m, rlo - m, rhi + m, -1);
  cover.init(qlo - m, qhi + m, rlo - m, rhi + m, 0);
  for (int64_t ply = 0; ply < n; ++ply) {
    int q = moves[2 * ply], r = moves[2 * ply + 1];
    int who = mover_after(ply);
    char msg[160];
    if (ply == 0) {
      if (q != 0 || r != 0) {
        std::snprintf(msg, sizeof msg, "ply 0: the opening must be the origin, got (%d, %d)", q, r);
        fail(HEXO_E_ILLEGAL, msg);
      }
    } else if (owner.at(q, r) >= 0 || !cover.at(q, r)) {
      std::snprintf(msg, sizeof msg, "ply %lld: (%d, %d) is not a legal placement",
                    (long long)ply, q, r);
      fail(HEXO_E_ILLEGAL, msg);
    }
    bool wins = completes_six(owner, q, r, who);
    owner.at(q, r) = int8_t(who);
    for (int dq = -kRadius; dq <= kRadius; ++dq)
      for (int dr = std::max(-kRadius, -kRadius - dq); dr <= std::min(kRadius, kRadius - dq); ++dr)
        cover.at(q + dq, r + dr) = 1;
    if (wins && allow_terminal && ply + 1 == n) {
      pos.winner = who;
      pos.mover = who;
      pos.moves_remaining = remaining_after(n);
      for (int qq = owner.q0; qq < owner.q0 + owner.nq; ++qq)
        for (int rr = owner.r0; rr < owner.r0 + owner.nr; ++rr)
          if (owner.at(qq, rr) >= 0) pos.stones.push_back({qq, rr, owner.at(qq, rr)});
      return pos;
    }
    if (wins) {
      std::snprintf(msg, sizeof msg, "ply %lld: (%d, %d) ends the game", (long long)ply, q, r);
      fail(ply + 1 == n ? HEXO_E_TERMINAL : HEXO_E_ILLEGAL,
           ply + 1 == n ? std::string("terminal position: the builder refuses it (") + msg + ")"
                        : std::string(msg) + "; later placements are on a terminal position");
    }
  }
  pos.mover = mover_after(n);
  pos.moves_remaining = remaining_after(n);
  if (n == 0) {
    pos.legal.push_back({0, 0});
    return pos;
  }
  for (int q = owner.q0; q < owner.q0 + owner.nq; ++q)
    for (int r = owner.r0; r < owner.r0 + owner.nr; ++r) {
      int o = owner.at(q, r);
      if (o >= 0) pos.stones.push_back({q, r, o});
      else if (cover.at(q, r)) pos.legal.push_back({q, r});
    }
  return pos;
}

// ------------------------------------------------------------- build

struct Graph {
  int64_t n_s = 0, n_w = 0, n_l = 0;
  int moves_remaining = 1;
  std::vector<int64_t> stone_own, window_feat, window_id, inc_stone, inc_window, inc_class;
  std::vector<int32_t> stone_q, stone_r;
  std::vector<int64_t> cell_nearest, radius_src, radius_dst, radius_orbit, radius_own,
      radius_on_axis;
  std::vector<int64_t> adj_src, adj_dst, adj_axis;
  std::vector<int64_t> dec_cell, dec_window, dec_class, act_class, act_empty;
  std::vector<int64_t> act_rev_local;  // window-major stable order of this position's decoder
  std::vector<float> tactical;
  // the dense action rows, legal-cell-major, then axis, then slot (18 per
  // cell): source window or -1, post-placement class, pre-placement status
  std::vector<int64_t> action_window, action_post1, action_status;
};

constexpr int64_t kStatusOwn = 0, kStatusOpp = 1, kStatusEmpty = 2, kStatusMixed = 3;
constexpr int kRowsPerCell = 18;

Graph build(const Position& pos) {
  const Vocab& V = vocab();
  Graph g;
  g.n_s = int64_t(pos.stones.size());
  g.n_l = int64_t(pos.legal.size());
  g.moves_remaining = pos.moves_remaining;
  if (g.n_l == 0) fail(HEXO_E_TERMINAL, "terminal position: the builder refuses it");

  int qlo = 0, qhi = 0, rlo = 0, rhi = 0;
  bool first = true;
  auto extend = [&](int q, int r) {
    if (first) qlo = qhi = q, rlo = rhi = r, first = false;
    qlo = std::min(qlo, q), qhi = std::max(qhi, q), rlo = std::min(rlo, r), rhi = std::max(rhi, r);
  };
  for (auto& s : pos.stones) extend(s[0], s[1]);
  for (auto& c : pos.legal) extend(c[0], c[1]);
  const int m = kRadius + kWin;  // a window through a legal cell reaches 5 further
  Grid<int32_t> sidx, lidx;
  Grid<uint8_t> wstart;
  sidx.init(qlo - m, qhi + m, rlo - m, rhi + m, -1);
  lidx.init(qlo - m, qhi + m, rlo - m, rhi + m, -1);
  wstart.init(qlo - m, qhi + m, rlo - m, rhi + m, 0);

  g.stone_own.resize(g.n_s);
  g.stone_q.resize(g.n_s);
  g.stone_r.resize(g.n_s);
  for (int64_t i = 0; i < g.n_s; ++i) {
    auto& s = pos.stones[i];
    g.stone_own[i] = s[2] != pos.mover;
    g.stone_q[i] = s[0];
    g.stone_r[i] = s[1];
    if (sidx.at(s[0], s[1]) >= 0) fail(HEXO_E_ARG, "duplicate stone coordinates");
    sidx.at(s[0], s[1]) = int32_t(i);
  }
  for (int64_t j = 0; j < g.n_l; ++j) lidx.at(pos.legal[j][0], pos.legal[j][1]) = int32_t(j);

  // Cell-node fields: radius edges destination-major; a stone ring scan in
  // ascending (q, r) of the stone visits sources in canonical index order.
  g.cell_nearest.resize(g.n_l);
  for (int64_t j = 0; j < g.n_l; ++j) {
    int cq = pos.legal[j][0], cr = pos.legal[j][1];
    if (sidx.at(cq, cr) >= 0) fail(HEXO_E_ARG, "a legal cell is occupied");
    int nearest = 9;
    for (int a = -kRadius; a <= kRadius; ++a)
      for (int b = std::max(-kRadius, -kRadius - a); b <= std::min(kRadius, kRadius - a); ++b) {
        int s = sidx.at(cq + a, cr + b);
        if (s < 0) continue;
        int dq = -a, dr = -b;
        int d = hexdist(dq, dr);
        nearest = std::min(nearest, d);
        g.radius_src.push_back(s);
        g.radius_dst.push_back(j);
        g.radius_orbit.push_back(V.orbit[dq + 12][dr + 12]);
        g.radius_own.push_back(g.stone_own[s]);
        g.radius_on_axis.push_back(dq == 0 || dr == 0 || dq + dr == 0);
      }
    if (g.n_s && nearest > kRadius) fail(HEXO_E_ARG, "a legal cell has no stone within radius 8");
    g.cell_nearest[j] = nearest;
  }
  // Adjacency: each destination's neighbours (src, axis), ordered by source.
  for (int64_t j = 0; j < g.n_l; ++j) {
    std::array<std::pair<int32_t, int>, 6> nb;
    int n = 0;
    for (int a = 0; a < 3; ++a)
      for (int t = -1; t <= 1; t += 2) {
        int s = lidx.get(pos.legal[j][0] + t * AQ[a], pos.legal[j][1] + t * AR[a], -1);
        if (s >= 0) nb[n++] = {s, a};
      }
    std::sort(nb.begin(), nb.begin() + n);
    for (int i = 0; i < n; ++i) {
      g.adj_dst.push_back(j);
      g.adj_src.push_back(nb[i].first);
      g.adj_axis.push_back(nb[i].second);
    }
  }

  // Live windows: every window through a stone, keyed (q*2^21 + r)*4 + axis,
  // which a row-major scan of start cells with axis innermost enumerates.
  for (auto& s : pos.stones)
    for (int a = 0; a < 3; ++a)
      for (int k = 0; k < kWin; ++k) wstart.at(s[0] - k * AQ[a], s[1] - k * AR[a]) |= uint8_t(1 << a);
  Grid<int32_t> widx;  // window index of (start, axis) at v[cell*3 + axis]
  widx.q0 = wstart.q0, widx.r0 = wstart.r0, widx.nq = wstart.nq, widx.nr = wstart.nr;
  widx.v.assign(wstart.v.size() * 3, -1);
  std::vector<int> wpattern, wown, wopp;
  int five_threats = 0, four_threats = 0;
  for (int q = wstart.q0; q < wstart.q0 + wstart.nq; ++q)
    for (int r = wstart.r0; r < wstart.r0 + wstart.nr; ++r) {
      uint8_t bits = wstart.at(q, r);
      if (!bits) continue;
      for (int a = 0; a < 3; ++a) {
        if (!(bits >> a & 1)) continue;
        int64_t w = int64_t(wpattern.size());
        widx.v[(size_t(q - widx.q0) * widx.nr + (r - widx.r0)) * 3 + a] = int32_t(w);
        int pattern = 0, own = 0, opp = 0;
        for (int k = 0; k < kWin; ++k) {
          int s = sidx.at(q + k * AQ[a], r + k * AR[a]);
          if (s < 0) continue;
          bool mine = g.stone_own[s] == 0;
          pattern += (mine ? 1 : 2) * V.pow3[k];
          own += mine;
          opp += !mine;
          g.inc_stone.push_back(s);
          g.inc_window.push_back(w);
          g.inc_class.push_back(-1);  // patched below once the pattern is known
        }
        for (int64_t e = int64_t(g.inc_class.size()) - own - opp, k = 0; k < kWin; ++k)
          if (V.digit(pattern, int(k)) != 0) g.inc_class[e++] = V.occ[pattern][k];
        if (own == 0 && opp == 5) ++five_threats;
        if (own == 0 && opp == 4) ++four_threats;
        wpattern.push_back(pattern);
        wown.push_back(own);
        wopp.push_back(opp);
        g.window_feat.push_back(V.rank[pattern]);
        g.window_id.insert(g.window_id.end(), {a, q, r});
      }
    }
  g.n_w = int64_t(wpattern.size());

  // Decoder incidence + action rows: legal-cell-major, axis, offset.
  g.act_empty.assign(size_t(g.n_l) * 3, 0);
  g.tactical.assign(size_t(g.n_l) * kTactical, 0.f);
  const float five_global = float(std::min(five_threats, kThreatCap)) / float(kThreatCap);
  const float four_global = float(std::min(four_threats, kThreatCap)) / float(kThreatCap);
  for (int64_t j = 0; j < g.n_l; ++j) {
    int cq = pos.legal[j][0], cr = pos.legal[j][1];
    bool win_now = false;
    int max_own = 0, max_opp = 0, own5 = 0, own4 = 0, opp5 = 0, opp4 = 0, kept = 0;
    for (int a = 0; a < 3; ++a)
      for (int k = 0; k < kWin; ++k) {
        int sq = cq - k * AQ[a], sr = cr - k * AR[a];
        int32_t w = widx.inside(sq, sr)
                        ? widx.v[(size_t(sq - widx.q0) * widx.nr + (sr - widx.r0)) * 3 + a]
                        : -1;
        int pre = w >= 0 ? wpattern[w] : 0, own = w >= 0 ? wown[w] : 0, opp = w >= 0 ? wopp[w] : 0;
        g.action_window.push_back(w);
        g.action_post1.push_back(V.post1[pre + V.pow3[k]][k]);
        g.action_status.push_back(w < 0 ? kStatusEmpty
                                  : own && opp ? kStatusMixed
                                  : own        ? kStatusOwn
                                               : kStatusOpp);
        if (w >= 0) {
          if (V.digit(pre, k) != 0) fail(HEXO_E_INTERNAL, "a legal action cell is occupied");
          int dc = V.dec[pre][k];
          int pc = V.post1[pre + V.pow3[k]][k];
          if (dc < 0 || pc < 0) fail(HEXO_E_INTERNAL, "decoder/action class out of vocabulary");
          g.dec_cell.push_back(j);
          g.dec_window.push_back(w);
          g.dec_class.push_back(dc);
          g.act_class.push_back(pc);
          ++kept;
        } else {
          g.act_empty[size_t(j) * 3 + std::min(k, kWin - 1 - k)] += 1;
        }
        if (opp == 0 && own == kWin - 1) win_now = true;
        max_own = std::max(max_own, own);
        max_opp = std::max(max_opp, opp);
        if (opp == 0 && own + 1 == 5) ++own5;
        if (opp == 0 && own + 1 == 4) ++own4;
        if (own == 0 && opp == 5) ++opp5;
        if (own == 0 && opp == 4) ++opp4;
      }
    float* t = &g.tactical[size_t(j) * kTactical];
    t[0] = win_now ? 1.f : 0.f;
    t[1] = float(max_own + 1) / float(kWin);
    t[2] = float(max_opp) / float(kWin);
    t[3] = float(own5) / 18.f;
    t[4] = float(own4) / 18.f;
    t[5] = float(opp5) / 18.f;
    t[6] = float(opp4) / 18.f;
    t[7] = five_global;
    t[8] = four_global;
    t[9] = (five_threats > 0 && opp5 == five_threats) ? 1.f : 0.f;
    t[10] = float(kept) / 18.f;
  }
  // Window-major stable order of the decoder entries (counting sort).
  {
    std::vector<int64_t> start(size_t(g.n_w) + 1, 0);
    for (int64_t w : g.dec_window) ++start[size_t(w) + 1];
    for (int64_t w = 0; w < g.n_w; ++w) start[size_t(w) + 1] += start[size_t(w)];
    g.act_rev_local.resize(g.dec_window.size());
    for (size_t e = 0; e < g.dec_window.size(); ++e)
      g.act_rev_local[size_t(start[size_t(g.dec_window[e])]++)] = int64_t(e);
  }
  return g;
}

// ------------------------------------------------------------- collate

struct Field {
  int32_t dtype;
  const void* data;
  int64_t numel;
};

}  // namespace

struct HexoBatch {
  int64_t n_pos = 0, max_t = 0, max_w = 0, n_cells = 0;
  std::vector<int64_t> stone_own, window_feat, window_id, moves_idx, inc_stone, inc_window,
      inc_class, stone_slot, window_slot, legal_offsets, cell_pos, cell_nearest, radius_src,
      radius_dst, radius_orbit, radius_own, radius_on_axis, adjacency_src, adjacency_dst,
      adjacency_axis, dec_cell, dec_window, dec_class, act_class, act_rev, act_empty;
  std::vector<int32_t> coords;
  std::vector<uint8_t> attn_valid, value_valid;
  std::vector<float> act_tactical;
  std::vector<int64_t> relay_cell_ptr, relay_window, relay_class, relay_win_ptr, relay_wcell,
      relay_cls_ptr, relay_ccell;
};

namespace {

template <typename F>
void parallel_for(int64_t n, int threads, F&& fn) {
  if (threads <= 0) threads = int(std::max(1u, std::thread::hardware_concurrency()));
  threads = int(std::min<int64_t>(threads, std::max<int64_t>(1, n)));
  if (threads <= 1) {
    for (int64_t i = 0; i < n; ++i) fn(i);
    return;
  }
  std::atomic<int64_t> next{0};
  std::vector<std::thread> pool;
  std::vector<std::string> errors{static_cast<size_t>(threads)};
  std::vector<int> codes(static_cast<size_t>(threads), 0);
  for (int t = 0; t < threads; ++t)
    pool.emplace_back([&, t] {
      try {
        for (int64_t i = next++; i < n; i = next++) fn(i);
      } catch (const Failure& f) {
        codes[size_t(t)] = f.code;
        errors[size_t(t)] = f.what();
        next = n;
      } catch (const std::exception& e) {
        codes[size_t(t)] = HEXO_E_INTERNAL;
        errors[size_t(t)] = e.what();
        next = n;
      }
    });
  for (auto& th : pool) th.join();
  for (int t = 0; t < threads; ++t)
    if (codes[size_t(t)]) fail(codes[size_t(t)], errors[size_t(t)]);
}

void relay_views(int64_t e, const int64_t* cell, const int64_t* win, const int64_t* cls,
                 int64_t n_windows, int64_t n_classes, std::vector<int64_t>& cell_ptr,
                 std::vector<int64_t>& window, std::vector<int64_t>& klass,
                 std::vector<int64_t>& win_ptr, std::vector<int64_t>& wcell,
                 std::vector<int64_t>& cls_ptr, std::vector<int64_t>& ccell) {
  int64_t max_cell = -1;
  for (int64_t i = 0; i < e; ++i) {
    if (cell[i] < 0) fail(HEXO_E_ARG, "dec_cell entries must be nonnegative");
    if (win[i] < 0 || win[i] >= n_windows)
      fail(HEXO_E_ARG, "dec_window entries must lie in [0, " + std::to_string(n_windows) + ")");
    if (cls[i] < 0 || cls[i] >= n_classes)
      fail(HEXO_E_ARG, "dec_class entries must lie in [0, " + std::to_string(n_classes) + ")");
    max_cell = std::max(max_cell, cell[i]);
  }
  // Stable counting sort by cell, then compact covered-cell labels.
  std::vector<int64_t> bucket(static_cast<size_t>(max_cell + 2), 0);
  std::vector<int64_t> order(static_cast<size_t>(e));
  for (int64_t i = 0; i < e; ++i) ++bucket[size_t(cell[i]) + 1];
  for (int64_t c = 0; c <= max_cell; ++c) bucket[size_t(c) + 1] += bucket[size_t(c)];
  std::vector<int64_t> pos_of(bucket.begin(), bucket.end() - 1);
  for (int64_t i = 0; i < e; ++i) order[size_t(pos_of[size_t(cell[i])]++)] = i;
  window.resize(size_t(e));
  klass.resize(size_t(e));
  std::vector<int64_t> edge_cell(static_cast<size_t>(e));
  cell_ptr.assign(1, 0);
  for (int64_t i = 0; i < e; ++i) {
    int64_t src = order[size_t(i)];
    window[size_t(i)] = win[src];
    klass[size_t(i)] = cls[src];
    if (i > 0 && cell[src] != cell[order[size_t(i - 1)]]) cell_ptr.push_back(i);
    edge_cell[size_t(i)] = int64_t(cell_ptr.size()) - 1;
  }
  if (e > 0) cell_ptr.push_back(e);
  auto by_key = [&](const std::vector<int64_t>& key, int64_t n_keys, std::vector<int64_t>& ptr,
                    std::vector<int64_t>& out) {
    ptr.assign(size_t(n_keys) + 1, 0);
    for (int64_t i = 0; i < e; ++i) ++ptr[size_t(key[size_t(i)]) + 1];
    for (int64_t k = 0; k < n_keys; ++k) ptr[size_t(k) + 1] += ptr[size_t(k)];
    std::vector<int64_t> fill(ptr.begin(), ptr.end() - 1);
    out.resize(size_t(e));
    for (int64_t i = 0; i < e; ++i) out[size_t(fill[size_t(key[size_t(i)])]++)] = edge_cell[size_t(i)];
  };
  by_key(window, n_windows, win_ptr, wcell);
  by_key(klass, n_classes, cls_ptr, ccell);
}

HexoBatch* collate(const std::vector<Graph>& gs, int threads) {
  auto* b = new HexoBatch();
  const int64_t p = int64_t(gs.size());
  if (p == 0) fail(HEXO_E_ARG, "empty batch");
  std::vector<int64_t> so(p + 1, 0), wo(p + 1, 0), co(p + 1, 0), io(p + 1, 0), dof(p + 1, 0),
      ro(p + 1, 0), ao(p + 1, 0);
  int64_t max_s = 0, max_w = 0;
  for (int64_t i = 0; i < p; ++i) {
    const Graph& g = gs[size_t(i)];
    so[i + 1] = so[i] + g.n_s;
    wo[i + 1] = wo[i] + g.n_w;
    co[i + 1] = co[i] + g.n_l;
    io[i + 1] = io[i] + int64_t(g.inc_stone.size());
    dof[i + 1] = dof[i] + int64_t(g.dec_cell.size());
    ro[i + 1] = ro[i] + int64_t(g.radius_src.size());
    ao[i + 1] = ao[i] + int64_t(g.adj_src.size());
    max_s = std::max(max_s, g.n_s);
    max_w = std::max(max_w, g.n_w);
  }
  b->n_pos = p;
  b->max_t = max_s + kGlobalRows;
  b->max_w = max_w + 1;
  b->n_cells = co[p];
  const int64_t T = b->max_t, MW = b->max_w;
  auto sz = [](int64_t n) { return size_t(n); };
  b->stone_own.resize(sz(so[p]));
  b->window_feat.resize(sz(wo[p]));
  b->window_id.resize(sz(3 * wo[p]));
  b->moves_idx.resize(sz(p));
  b->inc_stone.resize(sz(io[p]));
  b->inc_window.resize(sz(io[p]));
  b->inc_class.resize(sz(io[p]));
  b->stone_slot.resize(sz(so[p]));
  b->coords.assign(sz(p * T * 2), 0);
  b->attn_valid.assign(sz(p * T), 0);
  b->window_slot.resize(sz(wo[p]));
  b->value_valid.assign(sz(p * MW), 0);
  b->legal_offsets = co;
  b->cell_pos.resize(sz(co[p]));
  b->cell_nearest.resize(sz(co[p]));
  for (auto* v : {&b->radius_src, &b->radius_dst, &b->radius_orbit, &b->radius_own, &b->radius_on_axis})
    v->resize(sz(ro[p]));
  for (auto* v : {&b->adjacency_src, &b->adjacency_dst, &b->adjacency_axis}) v->resize(sz(ao[p]));
  for (auto* v : {&b->dec_cell, &b->dec_window, &b->dec_class, &b->act_class, &b->act_rev})
    v->resize(sz(dof[p]));
  b->act_empty.resize(sz(3 * co[p]));
  b->act_tactical.resize(sz(kTactical * co[p]));

  parallel_for(p, threads, [&](int64_t i) {
    const Graph& g = gs[size_t(i)];
    b->moves_idx[sz(i)] = g.moves_remaining - 1;
    for (int64_t s = 0; s < g.n_s; ++s) {
      b->stone_own[sz(so[i] + s)] = g.stone_own[sz(s)];
      b->stone_slot[sz(so[i] + s)] = i * T + kGlobalRows + s;
      b->coords[sz((i * T + kGlobalRows + s) * 2)] = g.stone_q[sz(s)];
      b->coords[sz((i * T + kGlobalRows + s) * 2 + 1)] = g.stone_r[sz(s)];
    }
    for (int64_t t = 0; t < kGlobalRows + g.n_s; ++t) b->attn_valid[sz(i * T + t)] = 1;
    for (int64_t w = 0; w < g.n_w; ++w) {
      b->window_feat[sz(wo[i] + w)] = g.window_feat[sz(w)];
      for (int k = 0; k < 3; ++k) b->window_id[sz(3 * (wo[i] + w) + k)] = g.window_id[sz(3 * w + k)];
      b->window_slot[sz(wo[i] + w)] = i * MW + 1 + w;
    }
    for (int64_t w = 0; w <= g.n_w; ++w) b->value_valid[sz(i * MW + w)] = 1;
    for (size_t e = 0; e < g.inc_stone.size(); ++e) {
      b->inc_stone[sz(io[i]) + e] = g.inc_stone[e] + so[i];
      b->inc_window[sz(io[i]) + e] = g.inc_window[e] + wo[i];
      b->inc_class[sz(io[i]) + e] = g.inc_class[e];
    }
    for (int64_t c = 0; c < g.n_l; ++c) {
      b->cell_pos[sz(co[i] + c)] = i;
      b->cell_nearest[sz(co[i] + c)] = g.cell_nearest[sz(c)];
      for (int k = 0; k < 3; ++k) b->act_empty[sz(3 * (co[i] + c) + k)] = g.act_empty[sz(3 * c + k)];
      for (int k = 0; k < kTactical; ++k)
        b->act_tactical[sz(kTactical * (co[i] + c) + k)] = g.tactical[sz(kTactical * c + k)];
    }
    for (size_t e = 0; e < g.radius_src.size(); ++e) {
      size_t o = sz(ro[i]) + e;
      b->radius_src[o] = g.radius_src[e] + so[i];
      b->radius_dst[o] = g.radius_dst[e] + co[i];
      b->radius_orbit[o] = g.radius_orbit[e];
      b->radius_own[o] = g.radius_own[e];
      b->radius_on_axis[o] = g.radius_on_axis[e];
    }
    for (size_t e = 0; e < g.adj_src.size(); ++e) {
      size_t o = sz(ao[i]) + e;
      b->adjacency_src[o] = g.adj_src[e] + co[i];
      b->adjacency_dst[o] = g.adj_dst[e] + co[i];
      b->adjacency_axis[o] = g.adj_axis[e];
    }
    for (size_t e = 0; e < g.dec_cell.size(); ++e) {
      size_t o = sz(dof[i]) + e;
      b->dec_cell[o] = g.dec_cell[e] + co[i];
      b->dec_window[o] = g.dec_window[e] + wo[i];
      b->dec_class[o] = g.dec_class[e];
      b->act_class[o] = g.act_class[e];
      b->act_rev[o] = g.act_rev_local[e] + dof[i];
    }
  });
  relay_views(dof[p], b->dec_cell.data(), b->dec_window.data(), b->dec_class.data(), wo[p],
              kDecClasses, b->relay_cell_ptr, b->relay_window, b->relay_class, b->relay_win_ptr,
              b->relay_wcell, b->relay_cls_ptr, b->relay_ccell);
  return b;
}

void write_err(char* err, int64_t len, const char* msg) {
  if (err && len > 0) {
    std::strncpy(err, msg, size_t(len) - 1);
    err[len - 1] = 0;
  }
}

template <typename F>
int32_t guarded(char* err, int64_t len, F&& fn) {
  try {
    fn();
    return HEXO_OK;
  } catch (const Failure& f) {
    write_err(err, len, f.what());
    return f.code;
  } catch (const std::exception& e) {
    write_err(err, len, e.what());
    return HEXO_E_INTERNAL;
  }
}

// ------------------------------------------------------------- wire format
//
// One live position as the versioned worker-to-batcher item of
// encoder.rs:539-621 (every integer little-endian):
//   magic "MANTIS\0\1", version u32, moves_remaining u8, 3 zero bytes,
//   counts u32 x 7 (stones, windows, incidences, legal, decoder, radius,
//   adjacency), then the per-position arrays in the order written below.

constexpr uint8_t kWireMagic[8] = {'M', 'A', 'N', 'T', 'I', 'S', 0, 1};
constexpr int64_t kWireHeader = 8 + 4 + 4 + 7 * 4;
constexpr uint32_t kReprVersion = 9;

struct WireOut {
  std::vector<uint8_t>& b;
  template <typename T>
  void put(T v) {
    uint8_t raw[sizeof(T)];
    std::memcpy(raw, &v, sizeof(T));  // little-endian host (x86-64, gfx hosts)
    b.insert(b.end(), raw, raw + sizeof(T));
  }
  template <typename T>
  void put_all(const std::vector<T>& v) {
    for (const T& x : v) put(x);
  }
};

// payload bytes after the header, or -1 on overflow
int64_t wire_payload(int64_t s, int64_t w, int64_t inc, int64_t l, int64_t d, int64_t r, int64_t a) {
  const int64_t n8 = s + 3 * w + w + 3 * inc + 3 * d + l + 5 * r + 3 * a + 3 * kRowsPerCell * l;
  if (n8 < 0 || n8 > (int64_t(1) << 58)) return -1;
  return 8 * n8 + 8 * s + 4 * int64_t(kTactical) * l;
}

void encode(const Graph& g, std::vector<uint8_t>& out) {
  const int64_t counts[7] = {g.n_s, g.n_w, int64_t(g.inc_stone.size()), g.n_l, int64_t(g.dec_cell.size()),
                             int64_t(g.radius_src.size()), int64_t(g.adj_src.size())};
  for (int64_t c : counts)
    if (c > int64_t(UINT32_MAX)) fail(HEXO_E_LIMIT, "a wire count exceeds u32");
  out.reserve(out.size() + size_t(kWireHeader + wire_payload(counts[0], counts[1], counts[2], counts[3], counts[4],
                                                             counts[5], counts[6])));
  WireOut o{out};
  out.insert(out.end(), kWireMagic, kWireMagic + 8);
  o.put(kReprVersion);
  o.put(uint8_t(g.moves_remaining));
  o.put(uint8_t(0)), o.put(uint8_t(0)), o.put(uint8_t(0));
  for (int64_t c : counts) o.put(uint32_t(c));
  o.put_all(g.stone_own);
  for (int64_t i = 0; i < g.n_s; ++i) o.put(int32_t(g.stone_q[size_t(i)])), o.put(int32_t(g.stone_r[size_t(i)]));
  o.put_all(g.window_feat);
  o.put_all(g.window_id);
  o.put_all(g.inc_stone), o.put_all(g.inc_window), o.put_all(g.inc_class);
  o.put_all(g.dec_cell), o.put_all(g.dec_window), o.put_all(g.dec_class);
  o.put_all(g.cell_nearest);
  o.put_all(g.radius_src), o.put_all(g.radius_dst), o.put_all(g.radius_orbit), o.put_all(g.radius_own),
      o.put_all(g.radius_on_axis);
  o.put_all(g.adj_src), o.put_all(g.adj_dst), o.put_all(g.adj_axis);
  o.put_all(g.action_window), o.put_all(g.action_post1), o.put_all(g.action_status);
  o.put_all(g.tactical);
}

struct WireIn {
  const uint8_t* p;
  int64_t n, at = 0;
  template <typename T>
  T get(const char* field) {
    if (n - at < int64_t(sizeof(T))) fail(HEXO_E_WIRE, std::string("truncated payload at ") + field);
    T v;
    std::memcpy(&v, p + at, sizeof(T));
    at += int64_t(sizeof(T));
    return v;
  }
  std::vector<int64_t> vec(int64_t count, const char* field) {
    std::vector<int64_t> v(static_cast<size_t>(count));
    for (auto& x : v) x = get<int64_t>(field);
    return v;
  }
};

[[noreturn]] void wire_fail(const std::string& msg) { fail(HEXO_E_WIRE, msg); }

std::string feature_error(const char* field, size_t i, int64_t v) {
  return std::string(field) + "[" + std::to_string(i) + "] has invalid feature " + std::to_string(v);
}

void check_range(const std::vector<int64_t>& v, int64_t lo, int64_t hi, const char* field) {
  for (size_t i = 0; i < v.size(); ++i)
    if (v[i] < lo || v[i] >= hi) wire_fail(feature_error(field, i, v[i]));
}

void check_index(const std::vector<int64_t>& v, int64_t upper, const char* field) {
  for (size_t i = 0; i < v.size(); ++i)
    if (v[i] < 0 || v[i] >= upper)
      wire_fail(std::string(field) + "[" + std::to_string(i) + "] index " + std::to_string(v[i]) +
                " is outside 0.." + std::to_string(upper));
}

// Parse and validate one item (the checks and their order of encoder.rs:666-941)
// into the graph build() would have produced.
Graph decode(const uint8_t* bytes, int64_t len) {
  const Vocab& V = vocab();
  WireIn in{bytes, len};
  if (len < 8 || std::memcmp(bytes, kWireMagic, 8) != 0) wire_fail("wrong magic");
  in.at = 8;
  const uint32_t version = in.get<uint32_t>("MODEL_REPR_VERSION");
  if (version != kReprVersion)
    wire_fail("MODEL_REPR_VERSION " + std::to_string(version) + " does not match " + std::to_string(kReprVersion));
  Graph g;
  const uint8_t mr = in.get<uint8_t>("moves_remaining");
  if (mr != 1 && mr != 2) wire_fail("moves_remaining must be 1 or 2, got " + std::to_string(mr));
  g.moves_remaining = mr;
  for (int i = 0; i < 3; ++i)
    if (in.get<uint8_t>("reserved bytes") != 0) wire_fail("reserved bytes are nonzero");
  const char* names[7] = {"stones", "windows", "incidences", "legal cells", "decoder incidences", "radius edges",
                          "adjacency edges"};
  int64_t c[7];
  for (int i = 0; i < 7; ++i) {
    c[i] = int64_t(in.get<uint32_t>(names[i]));
    // every count is capped at the item length before anything is sized by it
    if (c[i] > len)
      wire_fail(std::string(names[i]) + " count " + std::to_string(c[i]) + " exceeds item length " +
                std::to_string(len));
  }
  const int64_t S = c[0], W = c[1], I = c[2], L = c[3], D = c[4], R = c[5], A = c[6];
  if (L == 0) wire_fail("a live position must have a legal cell");
  const int64_t payload = wire_payload(S, W, I, L, D, R, A);
  if (payload < 0) wire_fail("payload length overflows");
  const int64_t expected = kWireHeader + payload;
  if (len < expected)
    wire_fail("truncated payload: header describes " + std::to_string(expected) + " bytes, got " +
              std::to_string(len));
  if (len > expected)
    wire_fail("trailing bytes: header describes " + std::to_string(expected) + " bytes, got " + std::to_string(len));
  g.n_s = S, g.n_w = W, g.n_l = L;

  g.stone_own = in.vec(S, "stone_own");
  check_range(g.stone_own, 0, 2, "stone_own");
  g.stone_q.resize(size_t(S)), g.stone_r.resize(size_t(S));
  for (int64_t i = 0; i < S; ++i) {
    const int32_t q = in.get<int32_t>("stone_qr.q"), r = in.get<int32_t>("stone_qr.r");
    if (q < INT16_MIN || q > INT16_MAX)
      wire_fail("stone_qr[" + std::to_string(i) + "].q is out of range: " + std::to_string(q));
    if (r < INT16_MIN || r > INT16_MAX)
      wire_fail("stone_qr[" + std::to_string(i) + "].r is out of range: " + std::to_string(r));
    if (std::abs(q) > kCoordLimit || std::abs(r) > kCoordLimit || std::abs(q + r) > kCoordLimit)
      wire_fail("stone_qr[" + std::to_string(i) + "] is not a valid engine coordinate: (" + std::to_string(q) +
                ", " + std::to_string(r) + ")");
    g.stone_q[size_t(i)] = q, g.stone_r[size_t(i)] = r;
  }
  g.window_feat = in.vec(W, "window_feat");
  check_range(g.window_feat, 0, kTernPatterns, "window_feat");
  g.window_id = in.vec(3 * W, "window_id");
  for (int64_t w = 0; w < W; ++w)
    if (g.window_id[size_t(3 * w)] < 0 || g.window_id[size_t(3 * w)] > 2)
      wire_fail(feature_error("window_id", size_t(w), g.window_id[size_t(3 * w)]));
  g.inc_stone = in.vec(I, "inc_stone");
  g.inc_window = in.vec(I, "inc_window");
  g.inc_class = in.vec(I, "inc_class");
  check_index(g.inc_stone, S, "inc_stone");
  check_index(g.inc_window, W, "inc_window");
  check_range(g.inc_class, 0, kTernOcc, "inc_class");
  g.dec_cell = in.vec(D, "dec_cell");
  g.dec_window = in.vec(D, "dec_window");
  g.dec_class = in.vec(D, "dec_class");
  check_index(g.dec_cell, L, "dec_cell");
  check_index(g.dec_window, W, "dec_window");
  check_range(g.dec_class, 0, kTernDec, "dec_class");
  g.cell_nearest = in.vec(L, "cell_nearest");
  check_range(g.cell_nearest, 0, kRadius + 2, "cell_nearest");
  g.radius_src = in.vec(R, "radius_src");
  g.radius_dst = in.vec(R, "radius_dst");
  g.radius_orbit = in.vec(R, "radius_orbit");
  g.radius_own = in.vec(R, "radius_own");
  g.radius_on_axis = in.vec(R, "radius_on_axis");
  check_index(g.radius_src, S, "radius_src");
  check_index(g.radius_dst, L, "radius_dst");
  check_range(g.radius_orbit, 0, 48, "radius_orbit");
  check_range(g.radius_own, 0, 2, "radius_own");
  check_range(g.radius_on_axis, 0, 2, "radius_on_axis");
  g.adj_src = in.vec(A, "adjacency_src");
  g.adj_dst = in.vec(A, "adjacency_dst");
  g.adj_axis = in.vec(A, "adjacency_axis");
  check_index(g.adj_src, L, "adjacency_src");
  check_index(g.adj_dst, L, "adjacency_dst");
  check_range(g.adj_axis, 0, 3, "adjacency_axis");
  g.action_window = in.vec(kRowsPerCell * L, "action_window_index");
  g.action_post1 = in.vec(kRowsPerCell * L, "action_post1_class");
  g.action_status = in.vec(kRowsPerCell * L, "action_pre_status");
  check_range(g.action_post1, 0, kTernPost1, "action_post1_class");
  // the kept rows, in order, are exactly the decoder incidences
  size_t edge = 0;
  for (size_t f = 0; f < g.action_window.size(); ++f) {
    const int64_t st = g.action_status[f], w = g.action_window[f];
    if (st < kStatusOwn || st > kStatusMixed) wire_fail(feature_error("action_pre_status", f, st));
    const bool kept = st != kStatusEmpty;
    if (kept != (w >= 0) || w >= W)
      wire_fail("action_window_index[" + std::to_string(f) + "]=" + std::to_string(w) + " disagrees with status " +
                std::to_string(st));
    if (kept) {
      if (edge >= g.dec_cell.size() || g.dec_cell[edge] != int64_t(f / kRowsPerCell) || g.dec_window[edge] != w)
        wire_fail("action row " + std::to_string(f) + " disagrees with decoder incidence " + std::to_string(edge));
      ++edge;
    }
  }
  if (edge != g.dec_cell.size())
    wire_fail(std::to_string(edge) + " kept action rows do not match " + std::to_string(g.dec_cell.size()) +
              " decoder incidences");
  g.tactical.resize(size_t(kTactical * L));
  for (size_t i = 0; i < g.tactical.size(); ++i) {
    const float v = in.get<float>("action_tactical");
    if (!std::isfinite(v) || v < 0.f || v > 1.f)
      wire_fail("action_tactical[" + std::to_string(i) + "] must be a finite value in [0, 1], got " +
                std::to_string(v));
    g.tactical[i] = v;
  }
  // the last tactical column is the nonempty-row fraction: demand bit equality
  for (int64_t j = 0; j < L; ++j) {
    int nonempty = 0;
    for (int k = 0; k < kRowsPerCell; ++k) nonempty += g.action_status[size_t(j * kRowsPerCell + k)] != kStatusEmpty;
    const float want = float(nonempty) / 18.f, got = g.tactical[size_t(j * kTactical + kTactical - 1)];
    if (std::memcmp(&want, &got, sizeof(float)) != 0)
      wire_fail("action_tactical[" + std::to_string(j) + "] nonempty column disagrees with the row statuses");
  }
  // the collated action fields: kept rows' classes, EMPTY rows per slot orbit
  g.act_empty.assign(size_t(3 * L), 0);
  for (size_t f = 0; f < g.action_status.size(); ++f) {
    const int k = int(f % kRowsPerCell) % kWin;
    if (g.action_status[f] == kStatusEmpty) ++g.act_empty[size_t(3 * int64_t(f / kRowsPerCell) + std::min(k, kWin - 1 - k))];
    else g.act_class.push_back(g.action_post1[f]);
  }
  std::vector<int64_t> start(size_t(W) + 1, 0);
  for (int64_t w : g.dec_window) ++start[size_t(w) + 1];
  for (int64_t w = 0; w < W; ++w) start[size_t(w) + 1] += start[size_t(w)];
  g.act_rev_local.resize(g.dec_window.size());
  for (size_t e = 0; e < g.dec_window.size(); ++e) g.act_rev_local[size_t(start[size_t(g.dec_window[e])]++)] = int64_t(e);
  return g;
}

}  // namespace

extern "C" {

int32_t hexo_repr_version(void) { return 9; }

int32_t hexo_build_batch_prefixes(int64_t n_games, const int16_t* moves_qr,
                                  const int64_t* move_offsets, const int64_t* ts,
                                  int32_t n_threads, HexoBatch** out, char* err,
                                  int64_t err_len) {
  return guarded(err, err_len, [&] {
    if (!out || n_games <= 0 || !move_offsets || !ts) fail(HEXO_E_ARG, "empty batch or null argument");
    *out = nullptr;
    for (int64_t i = 0; i < n_games; ++i) {
      int64_t len = move_offsets[i + 1] - move_offsets[i];
      if (len < 0 || ts[i] < 0 || ts[i] > len)
        fail(HEXO_E_ARG, "prefix length " + std::to_string(ts[i]) + " outside game " +
                             std::to_string(i) + " of length " + std::to_string(len));
    }
    (void)vocab();
    std::vector<Graph> graphs(static_cast<size_t>(n_games));
    parallel_for(n_games, n_threads, [&](int64_t i) {
      try {
        Position pos = replay(moves_qr + 2 * move_offsets[i], ts[i]);
        graphs[size_t(i)] = build(pos);
      } catch (const Failure& f) {
        fail(f.code, "game " + std::to_string(i) + ": " + f.what());
      }
    });
    *out = collate(graphs, n_threads);
  });
}

int32_t hexo_batch_scalars(const HexoBatch* b, int64_t* n_pos, int64_t* max_t, int64_t* max_w,
                           int64_t* n_cells) {
  if (!b) return HEXO_E_ARG;
  if (n_pos) *n_pos = b->n_pos;
  if (max_t) *max_t = b->max_t;
  if (max_w) *max_w = b->max_w;
  if (n_cells) *n_cells = b->n_cells;
  return HEXO_OK;
}

int32_t hexo_batch_field(const HexoBatch* b, const char* name, const void** data, int64_t* numel) {
  if (!b || !name) return 0;
  const std::pair<const char*, const std::vector<int64_t>*> i64[] = {
      {"stone_own", &b->stone_own}, {"window_feat", &b->window_feat},
      {"window_id", &b->window_id}, {"moves_idx", &b->moves_idx},
      {"inc_stone", &b->inc_stone}, {"inc_window", &b->inc_window},
      {"inc_class", &b->inc_class}, {"stone_slot", &b->stone_slot},
      {"window_slot", &b->window_slot}, {"legal_offsets", &b->legal_offsets},
      {"cell_pos", &b->cell_pos}, {"cell_nearest", &b->cell_nearest},
      {"radius_src", &b->radius_src}, {"radius_dst", &b->radius_dst},
      {"radius_orbit", &b->radius_orbit}, {"radius_own", &b->radius_own},
      {"radius_on_axis", &b->radius_on_axis}, {"adjacency_src", &b->adjacency_src},
      {"adjacency_dst", &b->adjacency_dst}, {"adjacency_axis", &b->adjacency_axis},
      {"dec_cell", &b->dec_cell}, {"dec_window", &b->dec_window},
      {"dec_class", &b->dec_class}, {"act_class", &b->act_class},
      {"act_rev", &b->act_rev}, {"act_empty", &b->act_empty},
      {"relay_cell_ptr", &b->relay_cell_ptr}, {"relay_window", &b->relay_window},
      {"relay_class", &b->relay_class}, {"relay_win_ptr", &b->relay_win_ptr},
      {"relay_wcell", &b->relay_wcell}, {"relay_cls_ptr", &b->relay_cls_ptr},
      {"relay_ccell", &b->relay_ccell},
  };
  for (auto& f : i64)
    if (!std::strcmp(f.first, name)) {
      if (data) *data = f.second->data();
      if (numel) *numel = int64_t(f.second->size());
      return HEXO_I64;
    }
  if (!std::strcmp(name, "coords")) {
    if (data) *data = b->coords.data();
    if (numel) *numel = int64_t(b->coords.size());
    return HEXO_I32;
  }
  if (!std::strcmp(name, "attn_valid") || !std::strcmp(name, "value_valid")) {
    const auto& v = name[0] == 'a' ? b->attn_valid : b->value_valid;
    if (data) *data = v.data();
    if (numel) *numel = int64_t(v.size());
    return HEXO_BOOL;
  }
  if (!std::strcmp(name, "act_tactical")) {
    if (data) *data = b->act_tactical.data();
    if (numel) *numel = int64_t(b->act_tactical.size());
    return HEXO_F32;
  }
  return 0;
}

void hexo_batch_free(HexoBatch* b) { delete b; }

int32_t hexo_relay_tables(int64_t e, const int64_t* dec_cell, const int64_t* dec_window,
                          const int64_t* dec_class, int64_t n_windows, int64_t n_classes,
                          int64_t* cell_ptr, int64_t* n_covered, int64_t* window, int64_t* cls,
                          int64_t* win_ptr, int64_t* wcell, int64_t* cls_ptr, int64_t* ccell,
                          char* err, int64_t err_len) {
  return guarded(err, err_len, [&] {
    if (e < 0 || n_windows < 0 || n_classes < 0) fail(HEXO_E_ARG, "negative size");
    std::vector<int64_t> cp, w, c, wp, wc, kp, kc;
    relay_views(e, dec_cell, dec_window, dec_class, n_windows, n_classes, cp, w, c, wp, wc, kp, kc);
    std::copy(cp.begin(), cp.end(), cell_ptr);
    *n_covered = int64_t(cp.size()) - 1;
    std::copy(w.begin(), w.end(), window);
    std::copy(c.begin(), c.end(), cls);
    std::copy(wp.begin(), wp.end(), win_ptr);
    std::copy(wc.begin(), wc.end(), wcell);
    std::copy(kp.begin(), kp.end(), cls_ptr);
    std::copy(kc.begin(), kc.end(), ccell);
  });
}

int32_t hexo_legal_moves(int64_t n_moves, const int16_t* moves_qr, int64_t cap, int16_t* legal_qr,
                         int64_t* n_legal, int32_t* mover, int32_t* moves_remaining, char* err,
                         int64_t err_len) {
  return guarded(err, err_len, [&] {
    Position pos = replay(moves_qr, n_moves);
    *n_legal = int64_t(pos.legal.size());
    if (int64_t(pos.legal.size()) > cap) fail(HEXO_E_ARG, "legal_qr capacity too small");
    for (size_t i = 0; i < pos.legal.size(); ++i) {
      legal_qr[2 * i] = int16_t(pos.legal[i][0]);
      legal_qr[2 * i + 1] = int16_t(pos.legal[i][1]);
    }
    if (mover) *mover = pos.mover;
    if (moves_remaining) *moves_remaining = pos.moves_remaining;
  });
}

int32_t hexo_random_game(int64_t n_stones, const double* u, int16_t* moves_qr, char* err,
                         int64_t err_len) {
  return guarded(err, err_len, [&] {
    if (n_stones < 1) fail(HEXO_E_ARG, "a game needs at least the opening stone");
    const int lim = 512;
    Grid<int8_t> owner, cover;
    owner.init(-lim, lim, -lim, lim, -1);
    cover.init(-lim, lim, -lim, lim, 0);
    int qlo = 0, qhi = 0, rlo = 0, rhi = 0;
    std::vector<std::array<int, 2>> choices;
    for (int64_t ply = 0; ply < n_stones; ++ply) {
      int who = mover_after(ply), q = 0, r = 0;
      if (ply > 0) {
        choices.clear();
        for (int cq = qlo - kRadius; cq <= qhi + kRadius; ++cq)
          for (int cr = rlo - kRadius; cr <= rhi + kRadius; ++cr)
            if (cover.at(cq, cr) && owner.at(cq, cr) < 0 && !completes_six(owner, cq, cr, who))
              choices.push_back({cq, cr});
        if (choices.empty()) fail(HEXO_E_INTERNAL, "no non-winning legal placement");
        double x = u[ply];
        if (!(x >= 0.0 && x < 1.0)) fail(HEXO_E_ARG, "draws must lie in [0, 1)");
        size_t k = std::min(choices.size() - 1, size_t(x * double(choices.size())));
        q = choices[k][0];
        r = choices[k][1];
      }
      if (std::abs(q) > lim - 2 * kRadius || std::abs(r) > lim - 2 * kRadius)
        fail(HEXO_E_LIMIT, "random game left the generator's board");
      owner.at(q, r) = int8_t(who);
      for (int dq = -kRadius; dq <= kRadius; ++dq)
        for (int dr = std::max(-kRadius, -kRadius - dq); dr <= std::min(kRadius, kRadius - dq); ++dr)
          cover.at(q + dq, r + dr) = 1;
      qlo = std::min(qlo, q), qhi = std::max(qhi, q), rlo = std::min(rlo, r), rhi = std::max(rhi, r);
      moves_qr[2 * ply] = int16_t(q);
      moves_qr[2 * ply + 1] = int16_t(r);
    }
  });
}

int32_t hexo_tables(int32_t* rank, int32_t* dec, int32_t* occ, int32_t* post1, int32_t* orbit,
                    float* pattern_counts) {
  return guarded(nullptr, 0, [&] {
    const Vocab& V = vocab();
    for (int p = 0; p < 729; ++p) {
      if (rank) rank[p] = V.rank[p];
      for (int s = 0; s < kWin; ++s) {
        if (dec) dec[p * kWin + s] = V.dec[p][s];
        if (occ) occ[p * kWin + s] = V.occ[p][s];
        if (post1) post1[p * kWin + s] = V.post1[p][s];
      }
    }
    if (orbit)
      for (int i = 0; i < 625; ++i) orbit[i] = V.orbit[i / 25][i % 25];
    if (pattern_counts) std::copy(V.counts.begin(), V.counts.end(), pattern_counts);
  });
}

int32_t hexo_encode_position(int64_t n_moves, const int16_t* moves_qr, uint8_t* out, int64_t cap, int64_t* len,
                             char* err, int64_t err_len) {
  return guarded(err, err_len, [&] {
    if (!len || n_moves < 0 || (n_moves > 0 && !moves_qr) || cap < 0 || (cap > 0 && !out))
      fail(HEXO_E_ARG, "null argument or negative size");
    std::vector<uint8_t> bytes;
    encode(build(replay(moves_qr, n_moves)), bytes);
    *len = int64_t(bytes.size());
    if (cap >= *len) std::memcpy(out, bytes.data(), bytes.size());
    else if (cap > 0) fail(HEXO_E_ARG, "output buffer of " + std::to_string(cap) + " bytes holds less than the " +
                                       std::to_string(*len) + "-byte item");
  });
}

int32_t hexo_decode_batch(int64_t n_items, const uint8_t* bytes, const int64_t* item_offsets, int32_t n_threads,
                          HexoBatch** out, char* err, int64_t err_len) {
  return guarded(err, err_len, [&] {
    if (!out || n_items <= 0 || !item_offsets || !bytes) fail(HEXO_E_ARG, "empty batch or null argument");
    *out = nullptr;
    for (int64_t i = 0; i < n_items; ++i)
      if (item_offsets[i] < 0 || item_offsets[i + 1] < item_offsets[i])
        fail(HEXO_E_ARG, "item offsets must be non-negative and ascending");
    (void)vocab();
    std::vector<Graph> graphs(static_cast<size_t>(n_items));
    parallel_for(n_items, n_threads, [&](int64_t i) {
      try {
        graphs[size_t(i)] = decode(bytes + item_offsets[i], item_offsets[i + 1] - item_offsets[i]);
      } catch (const Failure& f) {
        fail(f.code, "item " + std::to_string(i) + ": " + f.what());
      }
    });
    *out = collate(graphs, n_threads);
  });
}

int32_t hexo_position_state(int64_t n_moves, const int16_t* moves_qr, int64_t cap, int16_t* legal_qr,
                            int64_t* n_legal, int32_t* mover, int32_t* moves_remaining, int32_t* winner,
                            int64_t* n_stones, char* err, int64_t err_len) {
  return guarded(err, err_len, [&] {
    if (!n_legal || n_moves < 0 || (n_moves > 0 && !moves_qr) || cap < 0 || (cap > 0 && !legal_qr))
      fail(HEXO_E_ARG, "null argument or negative size");
    Position pos = replay(moves_qr, n_moves, true);
    *n_legal = int64_t(pos.legal.size());
    if (int64_t(pos.legal.size()) > cap) fail(HEXO_E_ARG, "legal_qr capacity too small");
    for (size_t i = 0; i < pos.legal.size(); ++i) {
      legal_qr[2 * i] = int16_t(pos.legal[i][0]);
      legal_qr[2 * i + 1] = int16_t(pos.legal[i][1]);
    }
    if (mover) *mover = pos.mover;
    if (moves_remaining) *moves_remaining = pos.moves_remaining;
    if (winner) *winner = pos.winner;
    if (n_stones) *n_stones = int64_t(pos.stones.size());
  });
}

}  // extern "C"

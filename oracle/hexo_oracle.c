/*
 * TEST INFRASTRUCTURE ONLY — the CPU oracle for the Hexo rules subset and the
 * MantisNet position encoder.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as a checker.
 *
 * Every routine is a deliberately literal restatement (brute-force loops, no
 * hashing, no incremental state) of the reference behaviour it cites, so that
 * it shares no structure with the product encoder it checks.
 *
 *   legal set / order ... crates/hexo-engine/README.md:47-50,111-115,197-200
 *   ternary tables ...... python/mantisnet/mantisnet/builder.py:88-229
 *   orbit48 ............. builder.py:41-84, encoder.rs:22-107
 *   build() ............. builder.py:486-642 (encoder.rs:1047-1355)
 *   cell_node_fields .... builder.py:427-483 (encoder.rs:943-1039)
 *   action tables ....... builder.py:262-424 (encoder.rs:1159-1355)
 *
 * Collation (offsets, padding, relay and action views) is restated in numpy
 * by oracle/encoder.py.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define WLEN 6
#define LEGAL_RADIUS 8
#define QSHIFT (1LL << 21)

static const int AX_Q[3] = {1, 0, 1};
static const int AX_R[3] = {0, 1, -1};

/* ------------------------------------------------------------------ tables */

static int pow3[WLEN];
static int tern_rev[729];
static int tern_rank[729];       /* 377 ranks, -1 for the empty pattern */
static int tern_dec[729][WLEN];  /* 726 classes, -1 elsewhere */
static int tern_occ[729][WLEN];  /* 1458 classes, -1 elsewhere */
static int tern_post1[729][WLEN];/* 729 classes, -1 elsewhere */
static int orbit_grid[25][25];   /* 48 classes for 1 <= d <= 12 */
static int tables_ready = 0;

static int digit_of(int p, int s) { return (p / pow3[s]) % 3; }

static int hexdist(int dq, int dr) {
  int a = dq < 0 ? -dq : dq, b = dr < 0 ? -dr : dr, c = dq + dr;
  if (c < 0) c = -c;
  int m = a > b ? a : b;
  return m > c ? m : c;
}

static int cmp_pair(int a0, int a1, int b0, int b1) {
  if (a0 != b0) return a0 < b0 ? -1 : 1;
  if (a1 != b1) return a1 < b1 ? -1 : 1;
  return 0;
}

/* rank `ids` (values in [0, n_ids)) by first appearance in ascending id order */
static void rerank(int joint[729][WLEN], int mask_kind, int out[729][WLEN]) {
  static int used[2187];
  memset(used, 0, sizeof(used));
  for (int p = 0; p < 729; ++p)
    for (int s = 0; s < WLEN; ++s) {
      int d = digit_of(p, s);
      int in = mask_kind == 0 ? (d == 0 && p != 0) : (d != 0);
      if (in) used[joint[p][s]] = 1;
    }
  int rank_of[2187], n = 0;
  for (int i = 0; i < 2187; ++i) rank_of[i] = used[i] ? n++ : -1;
  for (int p = 0; p < 729; ++p)
    for (int s = 0; s < WLEN; ++s) {
      int d = digit_of(p, s);
      int in = mask_kind == 0 ? (d == 0 && p != 0) : (d != 0);
      out[p][s] = in ? rank_of[joint[p][s]] : -1;
    }
}

/* 12 D6 images of a displacement: 6 rotations of it and of its reflection;
 * canonical form is the lexicographic minimum (builder.py:41-57). */
static void canon_disp(int q, int r, int* cq, int* cr) {
  int bq = q, br = r;
  for (int refl = 0; refl < 2; ++refl) {
    int iq = refl ? r : q, ir = refl ? q : r;
    for (int k = 0; k < 6; ++k) {
      if (cmp_pair(iq, ir, bq, br) < 0) { bq = iq; br = ir; }
      int nq = -ir, nr = iq + ir;
      iq = nq; ir = nr;
    }
  }
  *cq = bq; *cr = br;
}

int oracle_init(void) {
  if (tables_ready) return 0;
  pow3[0] = 1;
  for (int s = 1; s < WLEN; ++s) pow3[s] = pow3[s - 1] * 3;
  for (int p = 0; p < 729; ++p) {
    int r = 0;
    for (int s = 0; s < WLEN; ++s) r += digit_of(p, WLEN - 1 - s) * pow3[s];
    tern_rev[p] = r;
  }
  /* pattern ranks: canonical = min(p, rev p), ranked ascending over p >= 1 */
  {
    int seen[729];
    memset(seen, 0, sizeof(seen));
    for (int p = 1; p < 729; ++p) {
      int c = p < tern_rev[p] ? p : tern_rev[p];
      seen[c] = 1;
    }
    int rank_of[729], n = 0;
    for (int c = 0; c < 729; ++c) rank_of[c] = seen[c] ? n++ : -1;
    if (n != 377) return 1;
    for (int p = 0; p < 729; ++p) {
      int c = p < tern_rev[p] ? p : tern_rev[p];
      tern_rank[p] = p == 0 ? -1 : rank_of[c];
    }
  }
  /* joint (pattern, slot) orbits under (p, s) -> (rev p, 5 - s) */
  {
    static int joint[729][WLEN];
    int nxt = 0;
    for (int p = 0; p < 729; ++p)
      for (int s = 0; s < WLEN; ++s) {
        int rp = tern_rev[p], rs = WLEN - 1 - s;
        if (cmp_pair(p, s, rp, rs) <= 0) joint[p][s] = nxt++;
        else joint[p][s] = joint[rp][rs];
      }
    if (nxt != 2187) return 2;
    rerank(joint, 0, tern_dec);
    rerank(joint, 1, tern_occ);
  }
  /* post-placement (post, slot) orbits over own-digit slots */
  {
    int nxt = 0;
    for (int p = 0; p < 729; ++p)
      for (int s = 0; s < WLEN; ++s) {
        if (digit_of(p, s) != 1) { tern_post1[p][s] = -1; continue; }
        int rp = tern_rev[p], rs = WLEN - 1 - s;
        if (cmp_pair(p, s, rp, rs) <= 0) tern_post1[p][s] = nxt++;
        else tern_post1[p][s] = tern_post1[rp][rs];
      }
    if (nxt != 729) return 3;
  }
  /* orbit48: representatives sorted by (distance, canonical q, canonical r) */
  {
    int reps[600][3], n = 0;
    for (int q = -12; q <= 12; ++q)
      for (int r = -12; r <= 12; ++r) {
        int d = hexdist(q, r);
        if (d < 1 || d > 12) continue;
        int cq, cr;
        canon_disp(q, r, &cq, &cr);
        int dup = 0;
        for (int i = 0; i < n; ++i)
          if (reps[i][0] == d && reps[i][1] == cq && reps[i][2] == cr) dup = 1;
        if (!dup) { reps[n][0] = d; reps[n][1] = cq; reps[n][2] = cr; ++n; }
      }
    if (n != 48) return 4;
    for (int q = -12; q <= 12; ++q)
      for (int r = -12; r <= 12; ++r) {
        orbit_grid[q + 12][r + 12] = -1;
        int d = hexdist(q, r);
        if (d < 1 || d > 12) continue;
        int cq, cr;
        canon_disp(q, r, &cq, &cr);
        int rank = 0;
        for (int i = 0; i < n; ++i) {
          int less = reps[i][0] < d ||
                     (reps[i][0] == d && cmp_pair(reps[i][1], reps[i][2], cq, cr) < 0);
          rank += less;
        }
        orbit_grid[q + 12][r + 12] = rank;
      }
  }
  tables_ready = 1;
  return 0;
}

/* Table export: pattern rank (729), dec/occ/post1 classes (729*6 each),
 * orbit48 (25*25, indexed [dq+12][dr+12]). */
int oracle_tables(int32_t* rank, int32_t* dec, int32_t* occ, int32_t* post1,
                  int32_t* orbit) {
  if (oracle_init()) return 1;
  for (int p = 0; p < 729; ++p) {
    rank[p] = tern_rank[p];
    for (int s = 0; s < WLEN; ++s) {
      dec[p * WLEN + s] = tern_dec[p][s];
      occ[p * WLEN + s] = tern_occ[p][s];
      post1[p * WLEN + s] = tern_post1[p][s];
    }
  }
  for (int i = 0; i < 25 * 25; ++i) orbit[i] = orbit_grid[i / 25][i % 25];
  return 0;
}

/* ------------------------------------------------------------------ rules */

static int stone_at(int n, const int32_t* sq, const int32_t* sr, int q, int r) {
  for (int i = 0; i < n; ++i)
    if (sq[i] == q && sr[i] == r) return i;
  return -1;
}

/* Legal cells in ascending (q, r): the empty cells within 8 of a stone; at
 * ply 0 only the origin (README.md:47-50, 111-115).  Returns the count, or -1
 * if `cap` is too small. */
int64_t oracle_legal(int32_t n, const int32_t* sq, const int32_t* sr,
                     int32_t* out_q, int32_t* out_r, int64_t cap) {
  if (n == 0) {
    if (cap < 1) return -1;
    out_q[0] = 0; out_r[0] = 0;
    return 1;
  }
  int qlo = sq[0], qhi = sq[0], rlo = sr[0], rhi = sr[0];
  for (int i = 1; i < n; ++i) {
    if (sq[i] < qlo) qlo = sq[i];
    if (sq[i] > qhi) qhi = sq[i];
    if (sr[i] < rlo) rlo = sr[i];
    if (sr[i] > rhi) rhi = sr[i];
  }
  int64_t count = 0;
  for (int q = qlo - LEGAL_RADIUS; q <= qhi + LEGAL_RADIUS; ++q)
    for (int r = rlo - LEGAL_RADIUS; r <= rhi + LEGAL_RADIUS; ++r) {
      int near = 0, occupied = 0;
      for (int i = 0; i < n; ++i) {
        int d = hexdist(q - sq[i], r - sr[i]);
        if (d == 0) occupied = 1;
        if (d <= LEGAL_RADIUS) near = 1;
      }
      if (near && !occupied) {
        if (count >= cap) return -1;
        out_q[count] = q; out_r[count] = r; ++count;
      }
    }
  return count;
}

/* Whether placing `owner` at (q, r) makes six or more in a row on some axis. */
int oracle_completes_six(int32_t n, const int32_t* sq, const int32_t* sr,
                         const int32_t* owner, int32_t q, int32_t r, int32_t who) {
  for (int a = 0; a < 3; ++a) {
    int run = 1;
    for (int sign = -1; sign <= 1; sign += 2)
      for (int k = 1; k < 6; ++k) {
        int i = stone_at(n, sq, sr, q + sign * k * AX_Q[a], r + sign * k * AX_R[a]);
        if (i < 0 || owner[i] != who) break;
        ++run;
      }
    if (run >= 6) return 1;
  }
  return 0;
}

/* ------------------------------------------------------------------ build */

typedef struct {
  /* capacities in, counts out */
  int64_t n_windows, n_inc, n_dec, n_radius, n_adj;
} OracleCounts;

static int64_t pack_key(int q, int r) { return (int64_t)q * QSHIFT + r; }

/* window key -> index by linear scan over the sorted live keys */
static int64_t find_window(const int64_t* keys, int64_t n, int64_t key) {
  for (int64_t i = 0; i < n; ++i)
    if (keys[i] == key) return i;
  return -1;
}

static int cmp_i64(const void* a, const void* b) {
  int64_t x = *(const int64_t*)a, y = *(const int64_t*)b;
  return x < y ? -1 : x > y;
}

static int cmp_triple(const void* a, const void* b) {
  const int64_t* x = (const int64_t*)a;
  const int64_t* y = (const int64_t*)b;
  for (int i = 0; i < 3; ++i)
    if (x[i] != y[i]) return x[i] < y[i] ? -1 : 1;
  return 0;
}

/*
 * One position's graph (builder.py:486-642).  Stones arrive in canonical
 * (q, r) order with owners; legal cells in engine order.  Output buffers are
 * caller-allocated with the bounds documented in oracle/encoder.py; `cnt`
 * holds those capacities on entry and the produced counts on return.
 * Returns 0, or a positive error code.
 */
int oracle_build(int32_t n_s, const int32_t* sq, const int32_t* sr,
                 const int32_t* owner, int32_t mover, int32_t n_l,
                 const int32_t* lq, const int32_t* lr,
                 OracleCounts* cnt,
                 int64_t* stone_own,
                 int64_t* window_feat, int64_t* window_id,
                 int64_t* inc_stone, int64_t* inc_window, int64_t* inc_class,
                 int64_t* cell_nearest,
                 int64_t* radius_src, int64_t* radius_dst, int64_t* radius_orbit,
                 int64_t* radius_own, int64_t* radius_on_axis,
                 int64_t* adj_src, int64_t* adj_dst, int64_t* adj_axis,
                 int64_t* dec_cell, int64_t* dec_window, int64_t* dec_class,
                 int64_t* act_window, int64_t* act_post1, int64_t* act_status,
                 float* act_tactical) {
  if (oracle_init()) return 100;
  if (n_l <= 0) return 101;
  const OracleCounts cap = *cnt;
  for (int i = 0; i < n_s; ++i) stone_own[i] = owner[i] != mover;

  /* --- cell-node fields (builder.py:427-483) */
  int64_t ne = 0;
  for (int c = 0; c < n_l; ++c) {
    int nearest = 9;
    for (int s = 0; s < n_s; ++s) {
      int dq = lq[c] - sq[s], dr = lr[c] - sr[s];
      int d = hexdist(dq, dr);
      if (n_s && d < nearest) nearest = d;
      if (d == 0) return 102;
      if (d <= LEGAL_RADIUS) {
        if (ne >= cap.n_radius) return 103;
        radius_src[ne] = s;
        radius_dst[ne] = c;
        radius_orbit[ne] = orbit_grid[dq + 12][dr + 12];
        radius_own[ne] = stone_own[s];
        radius_on_axis[ne] = (dq == 0 || dr == 0 || dq + dr == 0);
        ++ne;
      }
    }
    if (n_s && nearest > LEGAL_RADIUS) return 104;
    cell_nearest[c] = n_s ? nearest : 9;
  }
  cnt->n_radius = ne;

  {
    int64_t (*adj)[3] = malloc(sizeof(int64_t[3]) * (size_t)(6 * n_l + 1));
    int64_t na = 0;
    for (int src = 0; src < n_l; ++src)
      for (int a = 0; a < 3; ++a)
        for (int sign = -1; sign <= 1; sign += 2) {
          int q = lq[src] + sign * AX_Q[a], r = lr[src] + sign * AX_R[a];
          for (int dst = 0; dst < n_l; ++dst)
            if (lq[dst] == q && lr[dst] == r) {
              adj[na][0] = dst; adj[na][1] = src; adj[na][2] = a; ++na;
            }
        }
    qsort(adj, (size_t)na, sizeof(int64_t[3]), cmp_triple);
    if (na > cap.n_adj) { free(adj); return 105; }
    for (int64_t i = 0; i < na; ++i) {
      adj_dst[i] = adj[i][0]; adj_src[i] = adj[i][1]; adj_axis[i] = adj[i][2];
    }
    cnt->n_adj = na;
    free(adj);
  }

  /* --- live windows: every (axis, start) through some stone, key-sorted */
  int64_t nw = 0;
  int64_t* keys = malloc(sizeof(int64_t) * (size_t)(18 * n_s + 1));
  for (int s = 0; s < n_s; ++s)
    for (int a = 0; a < 3; ++a)
      for (int k = 0; k < WLEN; ++k)
        keys[nw++] = pack_key(sq[s] - k * AX_Q[a], sr[s] - k * AX_R[a]) * 4 + a;
  qsort(keys, (size_t)nw, sizeof(int64_t), cmp_i64);
  {
    int64_t u = 0;
    for (int64_t i = 0; i < nw; ++i)
      if (u == 0 || keys[u - 1] != keys[i]) keys[u++] = keys[i];
    nw = u;
  }
  if (nw > cap.n_windows) { free(keys); return 106; }
  int* wpattern = malloc(sizeof(int) * (size_t)(nw + 1));
  int64_t ninc = 0;
  for (int64_t w = 0; w < nw; ++w) {
    int a = (int)(keys[w] & 3);
    int64_t packed = keys[w] >> 2;
    /* invert the packing: r in (-2^20, 2^20) */
    int64_t q = packed / QSHIFT, rem = packed % QSHIFT;
    if (rem < 0) { rem += QSHIFT; q -= 1; }
    if (rem >= QSHIFT / 2) { rem -= QSHIFT; q += 1; }
    int pattern = 0;
    int occupant[WLEN];
    for (int j = 0; j < WLEN; ++j) {
      int cq = (int)q + j * AX_Q[a], cr = (int)rem + j * AX_R[a];
      int i = stone_at(n_s, sq, sr, cq, cr);
      occupant[j] = i;
      if (i >= 0) pattern += (stone_own[i] == 0 ? 1 : 2) * pow3[j];
    }
    wpattern[w] = pattern;
    window_feat[w] = tern_rank[pattern];
    window_id[3 * w + 0] = a;
    window_id[3 * w + 1] = q;
    window_id[3 * w + 2] = rem;
    for (int j = 0; j < WLEN; ++j)
      if (occupant[j] >= 0) {
        if (ninc >= cap.n_inc) { free(keys); free(wpattern); return 107; }
        inc_stone[ninc] = occupant[j];
        inc_window[ninc] = w;
        inc_class[ninc] = tern_occ[pattern][j];
        if (inc_class[ninc] < 0) { free(keys); free(wpattern); return 108; }
        ++ninc;
      }
  }
  cnt->n_windows = nw;
  cnt->n_inc = ninc;

  /* --- decoder incidence and action rows: legal-cell-major, axis, offset */
  int64_t nd = 0;
  int five_ids_cap = (int)nw + 1;
  int64_t* five_ids = malloc(sizeof(int64_t) * (size_t)five_ids_cap);
  int64_t* four_ids = malloc(sizeof(int64_t) * (size_t)five_ids_cap);
  int n_five = 0, n_four = 0;
  /* first pass: the global opponent-threat census from the row table
   * (builder.py:368-373 deduplicates threat windows over every row) */
  for (int c = 0; c < n_l; ++c)
    for (int a = 0; a < 3; ++a)
      for (int k = 0; k < WLEN; ++k) {
        int sq0 = lq[c] - k * AX_Q[a], sr0 = lr[c] - k * AX_R[a];
        int own = 0, opp = 0;
        for (int j = 0; j < WLEN; ++j) {
          int i = stone_at(n_s, sq, sr, sq0 + j * AX_Q[a], sr0 + j * AX_R[a]);
          if (i >= 0) { if (stone_own[i] == 0) ++own; else ++opp; }
        }
        if (own == 0 && (opp == 5 || opp == 4)) {
          int64_t w = find_window(keys, nw, pack_key(sq0, sr0) * 4 + a);
          int64_t* ids = opp == 5 ? five_ids : four_ids;
          int* n = opp == 5 ? &n_five : &n_four;
          int dup = 0;
          for (int i = 0; i < *n; ++i) if (ids[i] == w) dup = 1;
          if (!dup) ids[(*n)++] = w;
        }
      }
  for (int c = 0; c < n_l; ++c) {
    int any_win = 0, max_own = 0, max_opp = 0, own5 = 0, own4 = 0;
    int opp5_hit = 0, opp4_hit = 0, kept_rows = 0;
    for (int a = 0; a < 3; ++a)
      for (int k = 0; k < WLEN; ++k) {
        int sq0 = lq[c] - k * AX_Q[a], sr0 = lr[c] - k * AX_R[a];
        int pre = 0, own = 0, opp = 0;
        for (int j = 0; j < WLEN; ++j) {
          int i = stone_at(n_s, sq, sr, sq0 + j * AX_Q[a], sr0 + j * AX_R[a]);
          if (i >= 0) {
            if (j == k) { free(keys); free(wpattern); free(five_ids); free(four_ids); return 109; }
            if (stone_own[i] == 0) { pre += pow3[j]; ++own; }
            else { pre += 2 * pow3[j]; ++opp; }
          }
        }
        int64_t row = ((int64_t)c * 3 + a) * WLEN + k;
        int status = own && !opp ? 0 : (opp && !own ? 1 : (own && opp ? 3 : 2));
        int64_t w = find_window(keys, nw, pack_key(sq0, sr0) * 4 + a);
        if ((w >= 0) != (status != 2)) {
          free(keys); free(wpattern); free(five_ids); free(four_ids); return 110;
        }
        act_window[row] = w;
        act_post1[row] = tern_post1[pre + pow3[k]][k];
        act_status[row] = status;
        if (act_post1[row] < 0) { free(keys); free(wpattern); free(five_ids); free(four_ids); return 111; }
        if (w >= 0) {
          if (nd >= cap.n_dec) { free(keys); free(wpattern); free(five_ids); free(four_ids); return 112; }
          dec_cell[nd] = c;
          dec_window[nd] = w;
          dec_class[nd] = tern_dec[wpattern[w]][k];
          if (dec_class[nd] < 0) { free(keys); free(wpattern); free(five_ids); free(four_ids); return 113; }
          ++nd;
          ++kept_rows;
        }
        if (!opp && own == WLEN - 1) any_win = 1;
        if (own > max_own) max_own = own;
        if (opp > max_opp) max_opp = opp;
        if (!opp && own + 1 == 5) ++own5;
        if (!opp && own + 1 == 4) ++own4;
        if (!own && opp == 5) ++opp5_hit;
        if (!own && opp == 4) ++opp4_hit;
      }
    float* t = act_tactical + (int64_t)c * 11;
    t[0] = (float)any_win;
    t[1] = (float)(max_own + 1) / 6.0f;
    t[2] = (float)max_opp / 6.0f;
    t[3] = (float)own5 / 18.0f;
    t[4] = (float)own4 / 18.0f;
    t[5] = (float)opp5_hit / 18.0f;
    t[6] = (float)opp4_hit / 18.0f;
    t[7] = (float)(n_five < 8 ? n_five : 8) / 8.0f;
    t[8] = (float)(n_four < 8 ? n_four : 8) / 8.0f;
    t[9] = (float)(n_five > 0 && opp5_hit == n_five);
    t[10] = (float)kept_rows / 18.0f;
  }
  cnt->n_dec = nd;
  free(keys);
  free(wpattern);
  free(five_ids);
  free(four_ids);
  return 0;
}

// Host-side metadata and work planner for the varlen and absorb operators.
//
// Pure C++17, no device calls: everything here runs (and is tested) on a CPU.
// It replaces the reference's Python metadata layer:
//   fa/interface.py:74-118          seqinfo -> cu_seqlens, validation
//   fa/chunk_indices.py:25-65       (seg, block) chunk tables
//   fa/chunk_indices.py:144-287     short / split / combine dispatch tables
//   ta/interface.py:92-138          validation, prepare_target_attn_indices
//   ta/chunk_indices.py:19-67       Q-major and K-major chunk tables
//
// Instead of (seg, block) pairs that every GPU program re-resolves through
// cu_seqlens, a plan holds 32-byte items with absolute token offsets, sorted
// longest-first (LPT) so that the long-tail tiles start first on a grid of
// many more workgroups than CUs.  Long key ranges are split; split items write
// compact partial rows (only the valid query rows) that a combine pass merges
// in a fixed order, so results are deterministic.
#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <numeric>
#include <string>
#include <vector>

#include "../../include/vafa.h"
#include "plan_params.h"

namespace vafa {

thread_local std::string g_last_error;

int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

namespace {

struct Item {
  int32_t v[VAFA_ITEM_INTS];
  int64_t cost;
};

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline int64_t round_up(int64_t a, int64_t b) { return cdiv(a, b) * b; }

// Number of key chunks for one query tile with `rows` valid rows against a
// segment of `lk` keys, and the chunk length (a multiple of `align`).
void key_split(int64_t rows, int64_t lk, const SplitPolicy &p, int64_t *ns_out,
               int64_t *chunk_out) {
  int64_t ns = 1;
  if (lk > 0) {
    if (rows <= p.decode_rows && lk >= p.decode_min_keys) {
      ns = std::min<int64_t>(std::max<int64_t>(cdiv(lk, p.decode_chunk), p.decode_min_split),
                             p.decode_max_split);
    } else if (lk > p.long_threshold) {
      ns = cdiv(lk, p.long_chunk);
    }
  }
  int64_t chunk = lk > 0 ? round_up(cdiv(lk, ns), p.align) : 0;
  if (chunk > 0) ns = cdiv(lk, chunk);
  *ns_out = ns;
  *chunk_out = chunk;
}

// Query and key tiles of a varlen plan.  A 256-row query tile (8-wave
// forward and dQ workgroups) shares every staged K/V tile among twice the
// queries: it pays off when most of the work (sum of Lq * Lk) lies in
// segments with more than 128 queries, and loses on decode-shaped batches,
// where one active wave per workgroup halves the key streams in flight per CU.
// 256-key dK/dV tiles pay off at D=128 (two waves per SIMD either way) when
// most of the work lies in segments with more than 128 keys; at D <= 64 the
// 4-wave kernel holds more waves per SIMD and stays.  Measured on the MI355X:
// configs[1] forward -2%, dK/dV -2.5%; configs[2] forward +10% with 256-row
// tiles; stage-1 replay (D=64) forward -6.6%, dK/dV +1.7% with 256-key tiles.
void varlen_tiles(const int64_t *cu_q, const int64_t *cu_k, int64_t n1, int64_t D, int64_t *bm,
                  int64_t *bk, int64_t *xcd_heads) {
  double work = 0.0, long_q = 0.0, long_k = 0.0;
  for (int64_t s = 0; s + 1 < n1; ++s) {
    const int64_t lq = cu_q[s + 1] - cu_q[s], lk = cu_k[s + 1] - cu_k[s];
    const double w = (double)lq * (double)lk;
    work += w;
    if (lq > kVarlenTile) long_q += w;
    if (lk > kVarlenTile) long_k += w;
  }
  *bm = D <= 128 && work > 0.0 && 2.0 * long_q >= work ? kVarlenWideTile : kVarlenTile;
  *bk = D == 128 && work > 0.0 && 2.0 * long_k >= work ? kVarlenWideTile : kVarlenTile;
  // Forward grid: when most of the work lies in segments of at most 128
  // queries (one query tile per key range), the H workgroups of an item run
  // on one XCD and read whole token rows of K/V together; otherwise the query
  // tiles of a segment run on one XCD and share its K/V in L2.  Measured on
  // the MI355X: configs[2] 5.58-5.70 -> 6.01-6.09 TB/s with grouped heads,
  // configs[1] forward 0.529 -> 0.548 ms (so it keeps the item-major grid).
  *xcd_heads = work > 0.0 && 2.0 * long_q < work ? 1 : 0;
}

void sort_lpt(std::vector<Item> &items) {
  std::stable_sort(items.begin(), items.end(),
                   [](const Item &a, const Item &b) { return a.cost > b.cost; });
}

// Items that read the same key range (same segment and split, different
// query tiles) form a bundle.  Bundles are assigned longest-first to the
// least-loaded XCD and the grid is laid out in rounds of kXcds slots, slot x
// running on XCD x, so the members of a bundle run back to back on one XCD
// and share its L2.  Empty slots are padded with no-op items (t0 == t1).
std::vector<Item> xcd_bundle(const std::vector<Item> &items) {
  std::vector<std::vector<Item>> bundles;
  std::vector<int64_t> cost;
  for (const Item &it : items) {
    // split items of one tile are emitted consecutively per (segment, split)
    bool joined = false;
    if (!bundles.empty()) {
      const Item &h = bundles.back().front();
      joined = h.v[5] == it.v[5] && h.v[6] == it.v[6] && h.v[2] == it.v[2] && h.v[3] == it.v[3];
    }
    if (!joined) {
      bundles.emplace_back();
      cost.push_back(0);
    }
    bundles.back().push_back(it);
    cost.back() += it.cost;
  }
  std::vector<size_t> order(bundles.size());
  std::iota(order.begin(), order.end(), 0);
  std::stable_sort(order.begin(), order.end(),
                   [&](size_t a, size_t b) { return cost[a] > cost[b]; });
  std::vector<std::vector<Item>> q(kXcds);
  std::vector<int64_t> load(kXcds, 0);
  for (size_t b : order) {
    const int x = (int)(std::min_element(load.begin(), load.end()) - load.begin());
    for (const Item &it : bundles[b]) q[x].push_back(it);
    load[x] += cost[b];
  }
  size_t rounds = 0;
  for (const auto &v : q) rounds = std::max(rounds, v.size());
  std::vector<Item> out;
  out.reserve(rounds * kXcds);
  const Item noop{{0, 0, 0, 0, -1, -1, 0, 1}, 0};
  for (size_t r = 0; r < rounds; ++r)
    for (int x = 0; x < kXcds; ++x) out.push_back(r < q[x].size() ? q[x][r] : noop);
  return out;
}

int64_t max_rows(const std::vector<Item> &comb) {
  // combine items start {q0, q1, ...} in every plan
  int64_t m = 0;
  for (const Item &it : comb) m = std::max<int64_t>(m, it.v[1] - it.v[0]);
  return m;
}

// Lays the sections out back to back: fwd, comb, kv, qt, then the varlen
// backward's dq, dqc, fkv, fcomb.
int emit(const std::vector<Item> &fwd, const std::vector<Item> &comb,
         const std::vector<Item> &kv, const std::vector<Item> &qt, const std::vector<Item> &dq,
         const std::vector<Item> &dqc, const std::vector<Item> &fkv,
         const std::vector<Item> &fcomb, int32_t *plan, int64_t cap, vafa_plan_info *info) {
  const std::vector<Item> *secs[] = {&fwd, &comb, &kv, &qt, &dq, &dqc, &fkv, &fcomb};
  int64_t *offs[] = {&info->off_fwd, &info->off_comb, &info->off_kv, &info->off_qt,
                     &info->off_dq, &info->off_dqc, &info->off_fkv, &info->off_fcomb};
  int64_t *counts[] = {&info->n_fwd, &info->n_comb, &info->n_kv, &info->n_qt,
                       &info->n_dq, &info->n_dqc, &info->n_fkv, &info->n_fcomb};
  int64_t off = 0;
  for (int i = 0; i < 8; ++i) {
    *offs[i] = off;
    *counts[i] = (int64_t)secs[i]->size();
    off += *counts[i] * VAFA_ITEM_INTS;
  }
  info->plan_ints = off;
  info->max_comb_rows = max_rows(comb);
  info->max_dqc_rows = max_rows(dqc);
  info->max_fcomb_rows = max_rows(fcomb);
  if (plan == nullptr) return VAFA_OK;
  if (cap < info->plan_ints)
    return fail(VAFA_ERR_CAPACITY, "plan buffer holds %lld int32, %lld needed",
                (long long)cap, (long long)info->plan_ints);
  int32_t *p = plan;
  for (const auto *sec : secs)
    for (const Item &it : *sec) {
      std::memcpy(p, it.v, sizeof(it.v));
      p += VAFA_ITEM_INTS;
    }
  return VAFA_OK;
}

int check_pair(const int64_t *cu_q, const int64_t *cu_k, int64_t n1) {
  if (n1 < 2) return fail(VAFA_ERR_VALUE, "cu_seqlens must have at least 2 elements");
  for (int64_t i = 0; i + 1 < n1; ++i) {
    if (cu_q[i + 1] < cu_q[i] || cu_k[i + 1] < cu_k[i])
      return fail(VAFA_ERR_VALUE, "cu_seqlens must be non-decreasing");
  }
  if (cu_q[0] != 0 || cu_k[0] != 0) return fail(VAFA_ERR_VALUE, "cu_seqlens[0] must be 0");
  if (cu_q[n1 - 1] > INT32_MAX || cu_k[n1 - 1] > INT32_MAX)
    return fail(VAFA_ERR_VALUE, "total tokens exceed int32 range");
  return VAFA_OK;
}

}  // namespace
}  // namespace vafa

using namespace vafa;

extern "C" {

const char *vafa_last_error(void) { return g_last_error.c_str(); }

int vafa_seqinfo_to_cu(const int64_t *seqinfo, int64_t n, int32_t *cu_out) {
  if (n <= 0) return fail(VAFA_ERR_VALUE, "seqinfo is empty (n_seg=0)");
  for (int64_t i = 0; i < n; ++i)
    if (seqinfo[i] < 0) return fail(VAFA_ERR_VALUE, "seqinfo contains negative values");
  int64_t acc = 0;
  cu_out[0] = 0;
  for (int64_t i = 0; i < n; ++i) {
    acc += seqinfo[i];
    if (acc > INT32_MAX)
      return fail(VAFA_ERR_VALUE, "total tokens %lld exceeds int32 range", (long long)acc);
    cu_out[i + 1] = (int32_t)acc;
  }
  return VAFA_OK;
}

int vafa_validate_cu(const int64_t *cu, int64_t n1, int64_t T, const char *name) {
  if (n1 < 2)
    return fail(VAFA_ERR_VALUE, "%s: must have at least 2 elements (n_seg+1 with n_seg>=1)",
                name);
  if (cu[0] != 0) return fail(VAFA_ERR_VALUE, "%s[0] must be 0, got %lld", name, (long long)cu[0]);
  if (cu[n1 - 1] != T)
    return fail(VAFA_ERR_VALUE, "%s[-1] must equal total tokens %lld, got %lld", name,
                (long long)T, (long long)cu[n1 - 1]);
  for (int64_t i = 0; i + 1 < n1; ++i)
    if (cu[i + 1] < cu[i])
      return fail(VAFA_ERR_VALUE, "%s must be non-decreasing (found negative segment length)",
                  name);
  return VAFA_OK;
}

int vafa_validate_cu_absorb(const int64_t *cu, int64_t n1, int64_t T, const char *name) {
  // same checks and order as vafa_validate_cu, with the absorb operator's texts
  if (n1 < 2)
    return fail(VAFA_ERR_VALUE, "%s: must be 1-D with len>=2, got (%lld,)", name,
                (long long)(n1 < 0 ? 0 : n1));
  if (cu[0] != 0) return fail(VAFA_ERR_VALUE, "%s[0] must be 0", name);
  if (cu[n1 - 1] != T)
    return fail(VAFA_ERR_VALUE, "%s[-1] must equal total tokens %lld, got %lld", name,
                (long long)T, (long long)cu[n1 - 1]);
  for (int64_t i = 0; i + 1 < n1; ++i)
    if (cu[i + 1] < cu[i]) return fail(VAFA_ERR_VALUE, "%s must be non-decreasing", name);
  return VAFA_OK;
}

int vafa_check_active_have_keys(const int64_t *cu_q, const int64_t *cu_k, int64_t n1) {
  for (int64_t i = 0; i + 1 < n1; ++i)
    if (cu_q[i + 1] - cu_q[i] > 0 && cu_k[i + 1] - cu_k[i] <= 0)
      return fail(VAFA_ERR_VALUE, "segments with q_len > 0 must have k_len > 0");
  return VAFA_OK;
}

int vafa_chunk_indices(const int64_t *cu, int64_t n1, int32_t BT, int32_t *out, int64_t cap,
                       int64_t *n_rows) {
  if (BT < 1) return fail(VAFA_ERR_ASSERT, "BT must be >= 1");
  if (n1 < 2) return fail(VAFA_ERR_ASSERT, "cu_seqlens must be 1-D with len >= 2");
  int64_t total = 0;
  for (int64_t i = 0; i + 1 < n1; ++i) {
    int64_t L = cu[i + 1] - cu[i];
    if (L > 0) total += cdiv(L, BT);
  }
  *n_rows = total;
  if (total > cap) return fail(VAFA_ERR_CAPACITY, "chunk table needs %lld rows", (long long)total);
  int64_t r = 0;
  for (int64_t i = 0; i + 1 < n1; ++i) {
    int64_t L = cu[i + 1] - cu[i];
    int64_t nb = L > 0 ? cdiv(L, BT) : 0;
    for (int64_t b = 0; b < nb; ++b, ++r) {
      out[2 * r] = (int32_t)i;
      out[2 * r + 1] = (int32_t)b;
    }
  }
  return VAFA_OK;
}

// Varlen plan.
//   fwd section   : one item per (segment, query tile, key chunk):
//                   {q0, q1, k0, k1, pbase, seg, split, nsplit}; pbase = -1
//                   writes O/LSE directly, otherwise partial rows
//                   pbase + r (r < q1-q0) hold this chunk's normalized O and LSE.
//   comb section  : one item per split query tile:
//                   {q0, q1, pbase, nsplit, seg, 0, 0, 0}; split s of the tile
//                   owns partial rows pbase + s*(q1-q0) + r.
//   kv section    : one item per (segment, key tile) for dK/dV:
//                   {k0, k1, q0, q1, seg, 0, 0, 0} with [q0,q1) the segment's
//                   whole query range.
//   dq, dqc       : the fwd and comb items of the segments that are not fused
//                   (same order, same partial rows): the dQ pass, which reuses
//                   the forward's split layout with its own partial buffer.
//   fkv section   : fused segments (at most kFusedMaxQ queries, D <=
//                   kFusedMaxD), one item per chunk of kFusedTiles 128-key
//                   tiles: {k0, k1, q0, q1, seg, pbase, chunk, nchunks}; the
//                   chunk's scaled fp32 dQ partial of query q lands in row
//                   pbase + (q - q0).
//   fcomb section : one item per fused segment, {q0, q1, pbase, nchunks, seg,
//                   0, 0, 0}: chunk t of the segment owns rows
//                   pbase + t*(q1-q0) + r (the comb layout), summed in order.
int vafa_plan_varlen(const int64_t *cu_q, const int64_t *cu_k, int64_t n1, int64_t H, int64_t D,
                     int32_t *plan, int64_t plan_cap, vafa_plan_info *info) {
  int rc = check_pair(cu_q, cu_k, n1);
  if (rc) return rc;
  const SplitPolicy &pol = kVarlenPolicy;
  int64_t BM = kVarlenTile, BK = kVarlenTile, xcd_heads = 0;
  varlen_tiles(cu_q, cu_k, n1, D, &BM, &BK, &xcd_heads);
  std::memset(info, 0, sizeof(*info));
  info->magic = VAFA_PLAN_MAGIC;
  info->kind = 1;
  info->n_seg = n1 - 1;
  info->T_q = cu_q[n1 - 1];
  info->T_k = cu_k[n1 - 1];
  info->H = H;
  info->q_tile = BM;
  info->k_tile = BK;
  info->xcd_heads = xcd_heads;
  std::vector<Item> fwd, comb, kv, fkv, fcomb;
  std::vector<char> fused(n1 > 1 ? n1 - 1 : 0, 0);
  int64_t prow = 0, fprow = 0;
  int64_t max_split = 1;
  for (int64_t s = 0; s + 1 < n1; ++s) {
    const int64_t q0 = cu_q[s], q1 = cu_q[s + 1], k0 = cu_k[s], k1 = cu_k[s + 1];
    const int64_t lq = q1 - q0, lk = k1 - k0;
    fused[s] = lq > 0 && lq <= kFusedMaxQ && lk >= kFusedMinK && D <= kFusedMaxD;
    for (int64_t t = q0; t < q1; t += BM) {
      const int64_t te = std::min(t + BM, q1), rows = te - t;
      int64_t ns, chunk;
      key_split(rows, lk, pol, &ns, &chunk);
      max_split = std::max(max_split, ns);
      if (ns <= 1) {
        Item it{{(int32_t)t, (int32_t)te, (int32_t)k0, (int32_t)k1, -1, (int32_t)s, 0, 1},
                lk + pol.item_overhead};
        fwd.push_back(it);
        continue;
      }
      Item c{{(int32_t)t, (int32_t)te, (int32_t)prow, (int32_t)ns, (int32_t)s, 0, 0, 0}, 0};
      comb.push_back(c);
      for (int64_t j = 0; j < ns; ++j) {
        const int64_t a = k0 + j * chunk, b = std::min(k1, a + chunk);
        Item it{{(int32_t)t, (int32_t)te, (int32_t)a, (int32_t)b, (int32_t)(prow + j * rows),
                 (int32_t)s, (int32_t)j, (int32_t)ns},
                (b - a) + pol.item_overhead};
        fwd.push_back(it);
      }
      prow += ns * rows;
    }
    // fused segments walk chunks of kFusedTiles 128-key tiles
    const int64_t bk = fused[s] ? (int64_t)kFusedTiles * kVarlenTile : BK;
    const int64_t ntiles = (lk + bk - 1) / bk;
    for (int64_t k = k0, j = 0; k < k1; k += bk, ++j) {
      const int64_t ke = std::min(k + bk, k1);
      if (fused[s]) {
        fkv.push_back(Item{{(int32_t)k, (int32_t)ke, (int32_t)q0, (int32_t)q1, (int32_t)s,
                            (int32_t)(fprow + j * lq), (int32_t)j, (int32_t)ntiles},
                           lq + pol.item_overhead});
      } else {
        kv.push_back(Item{{(int32_t)k, (int32_t)ke, (int32_t)q0, (int32_t)q1, (int32_t)s, 0, 0, 0},
                          lq + pol.item_overhead});
      }
    }
    if (fused[s] && ntiles > 0) {
      fcomb.push_back(Item{{(int32_t)q0, (int32_t)q1, (int32_t)fprow, (int32_t)ntiles,
                            (int32_t)s, 0, 0, 0}, 0});
      fprow += ntiles * lq;
    }
  }
  sort_lpt(fwd);
  sort_lpt(kv);
  sort_lpt(fkv);
  std::vector<Item> dq, dqc;
  for (const Item &it : fwd)
    if (!fused[it.v[5]]) dq.push_back(it);
  for (const Item &it : comb)
    if (!fused[it.v[4]]) dqc.push_back(it);
  info->n_part_rows = prow;
  info->n_fpart_rows = fprow;
  info->max_split = max_split;
  return emit(fwd, comb, kv, {}, dq, dqc, fkv, fcomb, plan, plan_cap, info);
}

// Absorb plan.  Query rows are (token, head) pairs; one item covers whole
// tokens [t0, t1) with (t1 - t0) * H <= kAbsorbRows.  A segment's tiles share
// one split of its key range.
//   fwd section : {t0, t1, k0, k1, pbase, seg, split, nsplit}; split items
//                 write projected partial rows pbase + r (r < t1-t0), each
//                 holding H x D_H fp32 outputs and H log2-domain LSEs.  The
//                 section is laid out XCD-aware (see xcd_bundle) and may hold
//                 no-op items {0, 0, 0, 0, -1, -1, 0, 1}.
//   comb section: {t0, t1, pbase, nsplit, seg, 0, 0, 0}.
//   kv section  : {k0, k1, t0, t1, seg, 0, 0, 0} key tiles for dX with the
//                 segment's whole token range [t0, t1).
//   qt section  : {t0, t1, k0, k1, -1, seg, 0, 1} unsplit token tiles with the
//                 segment's whole key range (backward dU pass).
int vafa_plan_absorb(const int64_t *cu_q, const int64_t *cu_k, int64_t n1, int64_t H,
                     int64_t D_KV, int64_t D_H, int32_t *plan, int64_t plan_cap,
                     vafa_plan_info *info) {
  int rc = check_pair(cu_q, cu_k, n1);
  if (rc) return rc;
  if (H < 1) return fail(VAFA_ERR_ASSERT, "H must be >= 1");
  (void)D_KV;
  (void)D_H;
  const int64_t TT = std::max<int64_t>(1, kAbsorbRows / H);
  const int64_t BK = kAbsorbKTile;
  // Key chunk of split segments, from the launch's total work: a chunk holds
  // kAbsorbSplitSlack times the average keys per resident forward workgroup
  // (never below kAbsorbPolicy.long_chunk), and only longer key ranges split.
  // Longest-first order starts such items at once, so they end within the
  // kernel; every extra item costs a prologue, an epilogue and a combine.
  SplitPolicy pol = kAbsorbPolicy;
  {
    int64_t work = 0;  // sum over segments of (token tiles x keys)
    for (int64_t s = 0; s + 1 < n1; ++s)
      if (cu_q[s + 1] > cu_q[s]) work += cdiv(cu_q[s + 1] - cu_q[s], TT) * (cu_k[s + 1] - cu_k[s]);
    const int64_t chunk = round_up(cdiv(kAbsorbSplitSlack * work, kAbsorbSlots), pol.align);
    pol.long_chunk = std::max<int64_t>(pol.long_chunk, chunk);
    pol.long_threshold = pol.long_chunk;
  }
  std::memset(info, 0, sizeof(*info));
  info->magic = VAFA_PLAN_MAGIC;
  info->kind = 2;
  info->n_seg = n1 - 1;
  info->T_q = cu_q[n1 - 1];
  info->T_k = cu_k[n1 - 1];
  info->H = H;
  info->q_tile = TT;
  info->k_tile = BK;
  std::vector<Item> fwd, comb, kv, qt;
  int64_t prow = 0, max_split = 1;
  for (int64_t s = 0; s + 1 < n1; ++s) {
    const int64_t q0 = cu_q[s], q1 = cu_q[s + 1], k0 = cu_k[s], k1 = cu_k[s + 1];
    const int64_t lq = q1 - q0, lk = k1 - k0;
    // one split decision per segment (its tiles share the key ranges)
    int64_t ns = 1, chunk = lk;
    if (lq > 0) key_split(std::min<int64_t>(lq, TT) * H, lk, pol, &ns, &chunk);
    max_split = std::max(max_split, ns);
    const int64_t seg_prow = prow;
    for (int64_t t = q0; t < q1; t += TT) {
      const int64_t te = std::min(t + TT, q1), ntok = te - t;
      const int64_t row_cost = round_up(ntok * H, 32);
      qt.push_back(Item{{(int32_t)t, (int32_t)te, (int32_t)k0, (int32_t)k1, -1, (int32_t)s, 0, 1},
                        (lk + pol.item_overhead) * row_cost});
      if (ns > 1) {
        Item c{{(int32_t)t, (int32_t)te, (int32_t)prow, (int32_t)ns, (int32_t)s, 0, 0, 0}, 0};
        comb.push_back(c);
        prow += ns * ntok;
      }
    }
    // forward items: split-major so that the tiles of one key range are adjacent
    for (int64_t j = 0; j < ns; ++j) {
      const int64_t a = ns > 1 ? k0 + j * chunk : k0;
      const int64_t b = ns > 1 ? std::min(k1, a + chunk) : k1;
      int64_t tile_prow = seg_prow;
      for (int64_t t = q0; t < q1; t += TT) {
        const int64_t te = std::min(t + TT, q1), ntok = te - t;
        const int64_t row_cost = round_up(ntok * H, 32);
        const int32_t pb = ns > 1 ? (int32_t)(tile_prow + j * ntok) : -1;
        fwd.push_back(Item{{(int32_t)t, (int32_t)te, (int32_t)a, (int32_t)b, pb, (int32_t)s,
                            (int32_t)j, (int32_t)ns},
                           ((b - a) + pol.item_overhead) * row_cost});
        tile_prow += ns * ntok;
      }
    }
    for (int64_t k = k0; k < k1; k += BK) {
      const int64_t ke = std::min(k + BK, k1);
      Item it{{(int32_t)k, (int32_t)ke, (int32_t)q0, (int32_t)q1, (int32_t)s, 0, 0, 0},
              (round_up(ke - k, 128) * round_up(lq * H, 32) + pol.item_overhead)};
      kv.push_back(it);
    }
  }
  fwd = xcd_bundle(fwd);
  sort_lpt(kv);
  // resident-row items first, so each dX kernel is launched over its own items
  const auto res_end = std::stable_partition(kv.begin(), kv.end(), [H](const Item &it) {
    return (int64_t)(it.v[3] - it.v[2]) * H <= kDxResidentRows;
  });
  info->n_kv_res = (int64_t)(res_end - kv.begin());
  sort_lpt(qt);
  info->n_part_rows = prow;
  info->max_split = max_split;
  return emit(fwd, comb, kv, qt, {}, {}, {}, {}, plan, plan_cap, info);
}

}  // extern "C"

// Randomized host test of the planner entry points of include/vafa.h
// (csrc/plan.cpp), built with AddressSanitizer and UndefinedBehaviorSanitizer
// by tests/test_host_sanitized.py.  For random segment layouts it checks that
// valid cu_seqlens plan without error, that every forward and key-tile item
// addresses tokens inside [0, T_q) x [0, T_k) (what the GPU kernels rely on),
// that a plan or chunk buffer one item too small is refused rather than
// overrun, and that corrupted cu_seqlens are rejected with an error code.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

#include "vafa.h"  // include/ (on the include path)

static int fails = 0;
#define CHECK(c)                                                                   \
  do {                                                                             \
    if (!(c)) {                                                                    \
      std::fprintf(stderr, "check failed at line %d: %s\n", __LINE__, #c);         \
      ++fails;                                                                     \
    }                                                                              \
  } while (0)

static std::vector<int64_t> cu_of(const std::vector<int64_t> &lens) {
  std::vector<int64_t> cu(lens.size() + 1, 0);
  for (size_t i = 0; i < lens.size(); ++i) cu[i + 1] = cu[i] + lens[i];
  return cu;
}

static int64_t draw_len(std::mt19937_64 &g) {
  switch (g() % 6) {
    case 0: return 0;
    case 1: return 1 + g() % 16;
    case 2: return 1 + g() % 300;
    case 3: return 1 + g() % 5000;
    case 4: return 1000 + g() % 40000;
    default: return (int64_t)(g() % 130);
  }
}

// Items [first, first + n) of a plan section: tokens of fields (a, a+1) in
// [0, Ta], of (b, b+1) in [0, Tb]; no-op items (all four zero) allowed.
static void check_ranges(const std::vector<int32_t> &plan, int64_t off, int64_t n, int a, int b,
                         int64_t Ta, int64_t Tb) {
  for (int64_t i = 0; i < n; ++i) {
    const int32_t *it = plan.data() + off + i * VAFA_ITEM_INTS;
    CHECK(0 <= it[a] && it[a] <= it[a + 1] && it[a + 1] <= Ta);
    CHECK(0 <= it[b] && it[b] <= it[b + 1] && it[b + 1] <= Tb);
  }
}

static void one_plan(bool absorb, const std::vector<int64_t> &cq, const std::vector<int64_t> &ck,
                     int64_t H, int64_t D) {
  vafa_plan_info info;
  const int64_t n1 = (int64_t)cq.size();
  int rc = absorb ? vafa_plan_absorb(cq.data(), ck.data(), n1, H, 256, D, nullptr, 0, &info)
                  : vafa_plan_varlen(cq.data(), ck.data(), n1, H, D, nullptr, 0, &info);
  CHECK(rc == VAFA_OK);
  if (rc != VAFA_OK) return;
  CHECK(info.plan_ints % VAFA_ITEM_INTS == 0 && info.T_q == cq.back() && info.T_k == ck.back());
  std::vector<int32_t> plan((size_t)info.plan_ints + 1, -7);
  if (info.plan_ints >= VAFA_ITEM_INTS) {
    vafa_plan_info small;
    rc = absorb ? vafa_plan_absorb(cq.data(), ck.data(), n1, H, 256, D, plan.data(),
                                   info.plan_ints - VAFA_ITEM_INTS, &small)
                : vafa_plan_varlen(cq.data(), ck.data(), n1, H, D, plan.data(),
                                   info.plan_ints - VAFA_ITEM_INTS, &small);
    CHECK(rc == VAFA_ERR_CAPACITY);
  }
  rc = absorb ? vafa_plan_absorb(cq.data(), ck.data(), n1, H, 256, D, plan.data(),
                                 info.plan_ints, &info)
              : vafa_plan_varlen(cq.data(), ck.data(), n1, H, D, plan.data(), info.plan_ints,
                                 &info);
  CHECK(rc == VAFA_OK);
  CHECK(plan.back() == -7);  // nothing written past plan_ints
  const int64_t Tq = cq.back(), Tk = ck.back();
  check_ranges(plan, info.off_fwd, info.n_fwd, 0, 2, Tq, Tk);  // {q0,q1,k0,k1}
  check_ranges(plan, info.off_kv, info.n_kv, 0, 2, Tk, Tq);    // {k0,k1,q0,q1}
  if (!absorb) {
    check_ranges(plan, info.off_dq, info.n_dq, 0, 2, Tq, Tk);
    check_ranges(plan, info.off_fkv, info.n_fkv, 0, 2, Tk, Tq);
  } else {
    check_ranges(plan, info.off_qt, info.n_qt, 0, 2, Tq, Tk);
  }
}

int main(int argc, char **argv) {
  const int iters = argc > 1 ? std::atoi(argv[1]) : 300;
  std::mt19937_64 g(argc > 2 ? std::strtoull(argv[2], nullptr, 10) : 12345);
  const int64_t Hs[] = {1, 2, 4, 8, 16, 32};
  const int64_t Ds[] = {16, 32, 64, 128, 256};
  for (int it = 0; it < iters; ++it) {
    const int n = 1 + (int)(g() % 40);
    std::vector<int64_t> lq(n), lk(n);
    for (int i = 0; i < n; ++i) {
      lq[i] = draw_len(g);
      lk[i] = g() % 3 == 0 ? lq[i] : draw_len(g);
    }
    const std::vector<int64_t> cq = cu_of(lq), ck = cu_of(lk);
    const int64_t n1 = (int64_t)cq.size();
    // metadata helpers
    CHECK(vafa_validate_cu(cq.data(), n1, cq.back(), "cu_seqlens_q") == VAFA_OK);
    CHECK(vafa_validate_cu_absorb(ck.data(), n1, ck.back(), "cu_seqlens_k") == VAFA_OK);
    std::vector<int32_t> cu32(lq.size() + 1);
    CHECK(vafa_seqinfo_to_cu(lq.data(), (int64_t)lq.size(), cu32.data()) == VAFA_OK);
    for (size_t i = 0; i < cq.size(); ++i) CHECK(cu32[i] == cq[i]);
    const int32_t BT = 1 + (int32_t)(g() % 128);
    int64_t rows = -1;
    int rc = vafa_chunk_indices(cq.data(), n1, BT, nullptr, 0, &rows);
    CHECK(rows >= 0 && (rows == 0 ? rc == VAFA_OK : rc == VAFA_ERR_CAPACITY));
    std::vector<int32_t> tab(2 * (size_t)rows + 1, -7);
    if (rows > 0) CHECK(vafa_chunk_indices(cq.data(), n1, BT, tab.data(), rows - 1, &rows) ==
                        VAFA_ERR_CAPACITY);
    CHECK(vafa_chunk_indices(cq.data(), n1, BT, tab.data(), rows, &rows) == VAFA_OK);
    CHECK(tab.back() == -7);
    // plans
    one_plan(false, cq, ck, Hs[g() % 6], Ds[g() % 5]);
    one_plan(true, cq, ck, Hs[g() % 4], Ds[g() % 4]);
    // corrupted cu_seqlens: rejected with an error code
    if (n > 0) {
      std::vector<int64_t> bad = cq;
      switch (g() % 3) {
        case 0: bad[0] = 1; break;
        case 1: bad[1 + g() % n] = -1 - (int64_t)(g() % 5); break;
        default: bad.back() += 1 + (int64_t)(g() % 3); break;
      }
      const bool ok_shape = bad[0] == 0;
      rc = vafa_validate_cu(bad.data(), n1, cq.back(), "cu_seqlens_q");
      CHECK(rc != VAFA_OK);
      vafa_plan_info info;
      rc = vafa_plan_varlen(bad.data(), ck.data(), n1, 4, 64, nullptr, 0, &info);
      if (!ok_shape || bad != cq) {
        bool monotone = true;
        for (size_t i = 0; i + 1 < bad.size(); ++i) monotone &= bad[i + 1] >= bad[i];
        if (!ok_shape || !monotone) CHECK(rc != VAFA_OK);
      }
    }
    std::vector<int64_t> neg(lq.begin(), lq.end());
    if (!neg.empty()) {
      neg[g() % neg.size()] = -1;
      CHECK(vafa_seqinfo_to_cu(neg.data(), (int64_t)neg.size(), cu32.data()) != VAFA_OK);
    }
  }
  // a single-element cu_seqlens (no segment) is refused everywhere
  {
    const int64_t z[1] = {0};
    int64_t rows = -1;
    int32_t cu1[1];
    vafa_plan_info info;
    CHECK(vafa_validate_cu(z, 1, 0, "cu_seqlens_q") != VAFA_OK);
    CHECK(vafa_chunk_indices(z, 1, 64, nullptr, 0, &rows) != VAFA_OK);
    CHECK(vafa_plan_varlen(z, z, 1, 4, 64, nullptr, 0, &info) != VAFA_OK);
    CHECK(vafa_plan_absorb(z, z, 1, 8, 256, 32, nullptr, 0, &info) != VAFA_OK);
    (void)cu1;
  }
  std::printf("plan_fuzz: %d iterations, %d failed checks\n", iters, fails);
  return fails == 0 ? 0 : 1;
}

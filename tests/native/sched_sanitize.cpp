// Host-only sanitizer run of the host scheduler (pkv_schedule.cpp, built here with g++ and
// -fsanitize=address,undefined; no device code): random decode steps through
// pkv_workqueue_size, pkv_build_workqueue, pkv_build_buckets and the split and route
// choices, every output buffer sized exactly to what the first call reports it needs, so
// that any write past it is caught.  Invalid inputs (negative lengths, short page lists)
// must come back as error codes.  The built queue must have the size pkv_workqueue_size
// predicted.  Usage: sched_sanitize [iterations]; prints "ok N, errors returned E".
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>
#include "pkv.h"

int main(int argc, char** argv) {
  const int iters = argc > 1 ? atoi(argv[1]) : 20000;
  std::mt19937 rng(12345);
  auto U = [&](int lo, int hi) { return std::uniform_int_distribution<int>(lo, hi)(rng); };
  const int sizes[] = {1, 5, 8, 16, 32, 64, 256};
  long ok = 0, errs = 0;
  for (int it = 0; it < iters; ++it) {
    const int count = U(0, it % 10 == 0 ? 300 : 12);
    const int ps = sizes[U(0, 6)];
    std::vector<int32_t> lens(count), ids(count), indptr(count + 1, 0), pages;
    bool bad = false;
    for (int r = 0; r < count; ++r) {
      int mode = U(0, 20);
      lens[r] = mode == 0 ? 0 : mode == 1 ? U(100000, 300000) : mode == 2 ? -U(1, 5) : U(1, 5000);
      if (lens[r] < 0) bad = true;
      ids[r] = U(0, 1000);
      int need = lens[r] > 0 ? (lens[r] + ps - 1) / ps : 1;
      if (U(0, 30) == 0) need = std::max(0, need - 1);  // short page list: an error or clamp
      for (int p = 0; p < need; ++p) pages.push_back(U(0, 1 << 20));
      indptr[r + 1] = (int32_t)pages.size();
    }
    const int hkv = 1 << U(0, 3);
    const int hq = hkv * (1 + U(0, 31));
    const int req = U(1, 64), autos = U(0, 1), policy = U(0, 1);
    int32_t tasks = -1, slots = -1;
    int st = pkv_workqueue_size(lens.data(), count, req, autos, hq, hkv, policy, &tasks, &slots);
    if (st == PKV_OK) {
      int32_t cols = 0, ntask = 0, nslots = 0;
      // First with zero capacities: sizes come back with PKV_ERR_CAPACITY (or OK if empty).
      std::vector<int32_t> sl(count), qi(count), oi(count), so(count + 1);
      st = pkv_build_workqueue(lens.data(), ids.data(), count, indptr.data(), pages.data(), ps,
                               req, autos, hq, hkv, policy, nullptr, 0, &cols, sl.data(),
                               qi.data(), oi.data(), nullptr, 0, &ntask, so.data(), &nslots);
      if (st == PKV_ERR_CAPACITY || st == PKV_OK) {
        std::vector<int32_t> table((size_t)count * cols), items((size_t)5 * ntask);
        st = pkv_build_workqueue(lens.data(), ids.data(), count, indptr.data(), pages.data(), ps,
                                 req, autos, hq, hkv, policy, table.data(), (int32_t)table.size(),
                                 &cols, sl.data(), qi.data(), oi.data(), items.data(), ntask,
                                 &ntask, so.data(), &nslots);
        if (st == PKV_OK) {
          if (ntask != tasks || nslots != slots) { printf("size mismatch it=%d\n", it); return 1; }
          ++ok;
        } else ++errs;
      } else ++errs;
    } else ++errs;
    // Buckets
    int32_t nb = 0; int64_t elems = 0;
    std::vector<int32_t> bl(count), br(count), bs(count), bc(count), sl2(count), qi2(count), oi2(count);
    st = pkv_build_buckets(lens.data(), ids.data(), count, indptr.data(), pages.data(), ps, req,
                           autos, U(0, 1) ? U(1, 4096) : 0, U(0, 1), U(0, 1), hkv, policy, &nb,
                           bl.data(), br.data(), bs.data(), bc.data(), sl2.data(), qi2.data(),
                           oi2.data(), nullptr, 0, &elems);
    if (st == PKV_ERR_CAPACITY || st == PKV_OK) {
      std::vector<int32_t> tabs((size_t)elems);
      st = pkv_build_buckets(lens.data(), ids.data(), count, indptr.data(), pages.data(), ps, req,
                             autos, 0, 1, 0, hkv, policy, &nb, bl.data(), br.data(), bs.data(),
                             bc.data(), sl2.data(), qi2.data(), oi2.data(), tabs.data(),
                             (int64_t)tabs.size(), &elems);
      (void)st;
    }
    // Router and split choices
    pkv_cost_model m;
    pkv_cost_model_preset(policy, &m);
    m.num_kv_heads = hkv; m.num_q_heads = hq;
    int32_t splits = 0; double ms = 0;
    if (count > 0 && !bad) {
      pkv_choose_adaptive_route(lens.data(), count, &m, &splits, &ms);
      pkv_choose_splits(lens.data(), count, req, autos, U(0, 1), hkv, policy);
      pkv_model_bucket_splits(lens.data(), count, hkv, policy);
      pkv_model_workqueue_splits(lens.data(), count, hkv, policy);
    }
  }
  printf("ok %ld, errors returned %ld\n", ok, errs);
  return 0;
}

// Differential check of the request packing in ft_runtime.cpp (host code,
// no GPU): random requests -- sorted and unsorted rows, ragged lengths,
// thresholds that keep all, some or none of a row -- are packed by
// pack_batch and compared with a plain scalar restatement of the staging
// format (rows in ascending token order with each proposal's index in the
// caller's row, the length-norm table, beam widths, and the per-step key
// bounds).  Requests with NaN / +inf logps or duplicate token ids must fail.
#include "ft_runtime.cpp"

#include <cstdio>
#include <memory>
#include <random>

namespace ftk {  // the device side is not linked here
hipError_t launch_tbs(const KArgs&, hipStream_t, hipEvent_t, hipEvent_t) { return hipErrorUnknown; }
hipError_t launch_root_dir(const KArgs&, RootEnt*, uint32_t, uint32_t, uint32_t, hipStream_t) {
  return hipErrorUnknown;
}
hipError_t clear_controls(uint8_t*, uint64_t, uint64_t, uint64_t, uint64_t, uint32_t, uint32_t,
                          hipStream_t) {
  return hipErrorUnknown;
}
hipError_t scratch_address(int, void**) { return hipErrorUnknown; }
int tbs_max_resident_blocks(int) { return 0; }
}  // namespace ftk

static int fails = 0;
#define CHECK(c, ...)                      \
  do {                                     \
    if (!(c)) {                            \
      if (fails++ < 10) {                  \
        std::printf("FAIL %s: ", #c);      \
        std::printf(__VA_ARGS__);          \
        std::printf("\n");                 \
      }                                    \
    }                                      \
  } while (0)

int main() {
  std::mt19937_64 g(12345);
  std::vector<uint8_t> H(8 << 20);
  std::vector<StagedReq> st(8);
  std::vector<std::pair<uint32_t, uint32_t>> tmp(4096);
  int cases = 0, rejected = 0;
  for (int c = 0; c < 3000; ++c) {
    const uint32_t T = 1 + g() % 6, K = 1 + g() % 70, n = 1 + g() % 4;
    const float thr = -(float)(g() % 12);
    const double sent = -(double)(g() % 30), alpha = (double)(g() % 6);
    std::vector<std::vector<uint32_t>> beams(n), ids(n);
    std::vector<std::vector<float>> lps(n);
    std::vector<ft_request> reqs(n);
    int expect_bad = 0;  // 1: NaN/inf, 2: duplicate
    for (uint32_t r = 0; r < n; ++r) {
      beams[r].resize(T);
      for (auto& b : beams[r]) b = 1 + g() % 9;
      ids[r].resize((size_t)T * K);
      lps[r].resize((size_t)T * K);
      for (uint32_t t = 0; t < T; ++t) {
        uint32_t v = (uint32_t)(g() % 5) | ((g() % 8 == 0) ? 0x80000000u : 0u);
        for (uint32_t k = 0; k < K; ++k) {
          v += 1 + (uint32_t)(g() % 4);
          ids[r][t * K + k] = v;
          lps[r][t * K + k] = -(float)(g() % 60) * 0.25f;
        }
        if (g() % 3 == 0 && r % 2 == 0)  // shuffle: an unsorted row (even requests only)
          std::shuffle(ids[r].begin() + t * K, ids[r].begin() + (t + 1) * K, g);
        if (K > 1 && g() % 40 == 0) {
          ids[r][t * K + 1] = ids[r][t * K];
          expect_bad = expect_bad ? expect_bad : 2;
        }
        if (g() % 60 == 0) {
          lps[r][t * K + g() % K] = (g() % 2) ? NAN : INFINITY;
          expect_bad = expect_bad ? expect_bad : 1;
        }
      }
      ft_request& q = reqs[r];
      std::memset(&q, 0, sizeof q);
      q.beams = beams[r].data();
      q.num_beams = T;
      q.num_steps = T;
      q.topk = K;
      q.topk_id = ids[r].data();
      q.topk_logp = lps[r].data();
      q.token_logp_threshold = thr;
      q.sent_logp_threshold = sent;
      q.length_norm = alpha;
    }
    for (auto& s : st) s = StagedReq();
    uint64_t used = 0, ostride = 0;
    StageLimits lim{64, 4096, 1000, 1u << 20};
    const int rc = pack_batch(reqs.data(), n, lim, H.data(), H.size(), st.data(), tmp.data(),
                              &used, &ostride);
    if (expect_bad) {
      CHECK(rc == FT_E_INPUT, "case %d: rc %d, expected an input error", c, rc);
      ++rejected;
      continue;
    }
    CHECK(rc == FT_OK, "case %d: rc %d %s", c, rc, g_err.c_str());
    if (rc) continue;
    ++cases;
    const DevReq* D = (const DevReq*)H.data();
    for (uint32_t r = 0; r < n; ++r) {
      const DevReq& d = D[r];
      const uint8_t* base = H.data() + d.in_off;
      CHECK(d.T == T && d.K == K && d.F == beams[r][T - 1], "case %d header", c);
      const double* lnf = (const double*)base;
      for (uint32_t dd = 0; dd <= T; ++dd)
        CHECK(lnf[dd] == std::pow(6.0 / (5.0 + dd), alpha), "case %d lnf", c);
      CHECK(std::memcmp(base + d.beams_off, beams[r].data(), 4 * T) == 0, "case %d beams", c);
      const uint32_t* rid = (const uint32_t*)(base + d.rid_off);
      const float* rlp = (const float*)(base + d.rlp_off);
      const uint16_t* rk = (const uint16_t*)(base + d.rk_off);
      const uint64_t* kb = (const uint64_t*)(base + d.kb_off);
      // the indices are staged iff some row is out of order; the kernel
      // reads [0, in_bytes) of the block, which must hold every array
      bool all_sorted = true;
      for (uint32_t t = 0; t < T; ++t)
        for (uint32_t k = 1; k < K; ++k)
          if (ids[r][t * K + k] <= ids[r][t * K + k - 1]) all_sorted = false;
      CHECK((d.rk_off == 0) == all_sorted, "case %d: rk_off %u, rows sorted %d", c, d.rk_off,
            (int)all_sorted);
      const uint64_t need = std::max<uint64_t>(
          {8ull * (T + 1), d.beams_off + 4ull * T, d.kb_off + 16ull * T, d.rid_off + 4ull * T * K,
           d.rlp_off + 4ull * T * K, d.rk_off ? d.rk_off + 2ull * T * K : 0ull});
      CHECK(d.in_bytes >= need && d.in_bytes % 16 == 0 && d.in_bytes < need + 16,
            "case %d: in_bytes %u for %lu", c, d.in_bytes, (unsigned long)need);
      if (r + 1 < n)
        CHECK(d.in_off + d.in_bytes <= D[r + 1].in_off, "case %d: blocks overlap", c);
      double s_lo = 0.0, s_hi = 0.0;
      for (uint32_t t = 0; t < T; ++t) {
        std::vector<std::pair<uint32_t, uint32_t>> e(K);
        for (uint32_t k = 0; k < K; ++k) e[k] = {ids[r][t * K + k], k};
        std::sort(e.begin(), e.end());
        double x_lo = 0.0, x_hi = 0.0;
        bool any = false;
        for (uint32_t p = 0; p < K; ++p) {
          CHECK(rid[t * K + p] == e[p].first &&
                    (d.rk_off ? (uint32_t)rk[t * K + p] : p) == e[p].second &&
                    rlp[t * K + p] == lps[r][t * K + e[p].second],
                "case %d row %u pos %u", c, t, p);
          const double x = (double)lps[r][t * K + p];
          if (x <= (double)thr) continue;
          if (!any || x < x_lo) x_lo = x;
          if (!any || x > x_hi) x_hi = x;
          any = true;
        }
        const double lo = std::max(sent, s_lo + x_lo), hi = s_hi + x_hi;
        CHECK(kb[2 * t] == host_norm_key(lo * lnf[t + 1]) &&
                  kb[2 * t + 1] == host_norm_key(hi * lnf[t + 1]),
              "case %d bounds of step %u", c, t);
        s_lo = lo;
        s_hi = hi;
      }
    }
  }
  // The streamed search's packing: plan_batch lays the batch out, then
  // pack_stream packs the requests and writes their ready words -- whole
  // requests, or the first 1 or 3 rows of every request before the rest.
  // The blocks must equal pack_batch's; each final word holds the row count
  // and whether the row indices are staged; a request with a NaN is
  // withdrawn (and only it -- the others stay ready), where pack_batch
  // fails.
  int streamed = 0;
  std::vector<uint8_t> H2(8 << 20);
  std::vector<StagedReq> st2(8);
  std::vector<unsigned long long> ready(8);
  for (int c = 0; c < 400; ++c) {
    const uint32_t T = 1 + g() % 6, K = 1 + g() % 300, n = 2 + g() % 7;
    std::vector<std::vector<uint32_t>> beams(n), ids(n);
    std::vector<std::vector<float>> lps(n);
    std::vector<ft_request> reqs(n);
    const uint32_t nan_req = (g() % 4 == 0) ? (uint32_t)(g() % n) : n;
    for (uint32_t r = 0; r < n; ++r) {
      beams[r].assign(T, 1 + (uint32_t)(g() % 9));
      ids[r].resize((size_t)T * K);
      lps[r].resize((size_t)T * K);
      for (uint32_t t = 0; t < T; ++t) {
        uint32_t v = (uint32_t)(g() % 5);
        for (uint32_t k = 0; k < K; ++k) {
          v += 1 + (uint32_t)(g() % 4);
          ids[r][t * K + k] = v;
          lps[r][t * K + k] = -(float)(g() % 60) * 0.25f;
        }
        if (g() % 3 == 0)
          std::shuffle(ids[r].begin() + t * K, ids[r].begin() + (t + 1) * K, g);
      }
      if (r == nan_req) lps[r][g() % ((size_t)T * K)] = NAN;
      ft_request& q = reqs[r];
      std::memset(&q, 0, sizeof q);
      q.beams = beams[r].data();
      q.num_beams = T;
      q.num_steps = T;
      q.topk = K;
      q.topk_id = ids[r].data();
      q.topk_logp = lps[r].data();
      q.token_logp_threshold = -5.0f;
      q.sent_logp_threshold = -20.0;
      q.length_norm = 2.0;
    }
    StageLimits lim{64, 4096, 1000, 1u << 20};
    uint64_t used = 0, used2 = 0, os = 0, os2 = 0;
    // (padding and unstaged row indices are left unwritten: start both alike)
    std::memset(H.data(), 0, 1 << 20);
    std::memset(H2.data(), 0, 1 << 20);
    for (auto& x : st) x = StagedReq();
    for (auto& x : st2) x = StagedReq();
    const int rc1 = pack_batch(reqs.data(), n, lim, H.data(), H.size(), st.data(), tmp.data(),
                               &used, &os);
    size_t first_bad = n;
    std::string msg;
    const int rc2 = plan_batch(reqs.data(), n, lim, H2.data(), H2.size(), st2.data(), &used2,
                               &os2, &first_bad, &msg);
    CHECK(rc2 == FT_OK && used2 == used, "stream case %d: plan rc %d", c, rc2);
    // the headers as launched: packing must leave them as they are (the
    // kernel copies them while the host packs), and they must fit
    std::vector<DevReq> planned((const DevReq*)H2.data(), (const DevReq*)H2.data() + n);
    for (uint32_t r = 0; r < n; ++r)
      CHECK(block_fits(used2, planned[r]), "stream case %d request %u: planned block", c, r);
    PackJob job;
    job.reqs = reqs.data();
    job.D = (DevReq*)H2.data();
    job.H = H2.data();
    job.staged = st2.data();
    job.ready = ready.data();
    job.tag = (unsigned long long)(c + 1) << 32;
    job.batch = n;
    job.head_rows = c % 3 == 0 ? 0u : c % 3 == 1 ? 1u : 3u;
    job.rc.assign(n, FT_OK);
    job.msg.resize(n);
    pack_stream(job, tmp.data());
    for (uint32_t r = 0; r < n; ++r) {
      const bool bad = r == nan_req;
      CHECK((job.rc[r] != FT_OK) == bad, "stream case %d request %u: rc %d", c, r, job.rc[r]);
      CHECK(std::memcmp(&job.D[r], &planned[r], sizeof(DevReq)) == 0,
            "stream case %d request %u: the launched header was rewritten", c, r);
      // the indices are staged (kReadyRk) iff pack_batch stages them
      const bool rk = rc1 == FT_OK && ((const DevReq*)H.data())[r].rk_off != 0;
      const unsigned long long want =
          bad ? kReadyWithdrawn
              : ((unsigned long long)T << kReadyRowsShift) | kReadyOk | (rk ? kReadyRk : 0u);
      if (rc1 == FT_OK || bad)
        CHECK(ready[r] == (job.tag | want), "stream case %d request %u: ready word %llx", c, r,
              ready[r]);
    }
    if (nan_req == n) {
      CHECK(rc1 == FT_OK, "stream case %d: pack_batch rc %d", c, rc1);
      // the blocks equal pack_batch's; its headers differ only in rk_off and
      // in_bytes, which it trims when no indices are staged
      const size_t hdr = align_up(n * sizeof(DevReq), 256);
      CHECK(std::memcmp(H.data() + hdr, H2.data() + hdr, used - hdr) == 0,
            "stream case %d: blocks differ", c);
      for (uint32_t r = 0; r < n; ++r) {
        DevReq x = ((const DevReq*)H.data())[r], y = planned[r];
        CHECK(x.rk_off == 0 || x.rk_off == y.rk_off, "stream case %d: rk_off", c);
        x.rk_off = y.rk_off = 0;
        x.in_bytes = y.in_bytes = 0;
        CHECK(std::memcmp(&x, &y, sizeof x) == 0, "stream case %d: headers differ", c);
      }
      ++streamed;
    } else {
      CHECK(rc1 == FT_E_INPUT, "stream case %d: pack_batch rc %d", c, rc1);
    }
  }
  // The row scan's SIMD variants against a scalar restatement (the ones
  // this host runs): random rows with NaN, +-inf, +-0, ids around 2^31,
  // equal and descending neighbours, thresholds inside and outside the
  // range, lengths around the vector widths.
  int scanned = 0;
  {
    struct Variant {
      const char* name;
      ScanRowFn fn;
      bool ok;
    } vars[] = {{"sse2", scan_row_sse2, true},
                {"avx2", scan_row_avx2, (bool)__builtin_cpu_supports("avx2")}};
    std::vector<uint32_t> id(80), oid(80);
    std::vector<float> lp(80), olp(80);
    const float specials[] = {NAN, INFINITY, -INFINITY, 0.0f, -0.0f, -1e-30f, 3.5f};
    for (int c = 0; c < 20000; ++c) {
      const uint32_t K = (uint32_t)(g() % 70);
      uint32_t v = (g() % 2) ? 0x7FFFFFF0u : (uint32_t)(g() % 100);
      for (uint32_t k = 0; k < K; ++k) {
        v += (uint32_t)(g() % 3);  // 0: an equal neighbour
        id[k] = (g() % 50 == 0) ? v - 5u : v;
        lp[k] = (g() % 25 == 0) ? specials[g() % 7] : -(float)(g() % 80) * 0.25f;
      }
      const float thr = (g() % 5 == 0) ? specials[g() % 7] : -(float)(g() % 25);
      bool bad = false, sorted = true;
      float lo = INFINITY, hi = -INFINITY;
      for (uint32_t k = 0; k < K; ++k) {
        bad = bad || std::isnan(lp[k]) || lp[k] == INFINITY;
        if (lp[k] > thr) {
          lo = std::min(lo, lp[k]);
          hi = std::max(hi, lp[k]);
        }
        if (k > 0 && id[k] <= id[k - 1]) sorted = false;
      }
      for (const Variant& w : vars) {
        if (!w.ok) continue;
        std::fill(oid.begin(), oid.end(), 0u);
        std::fill(olp.begin(), olp.end(), 0.0f);
        const RowScan sc = w.fn(id.data(), lp.data(), K, thr, oid.data(), olp.data());
        CHECK(sc.bad == bad, "scan %s case %d: bad", w.name, c);
        if (!bad) {
          CHECK(sc.sorted == sorted, "scan %s case %d: sorted", w.name, c);
          // +0 and -0 may come out either way; the bounds treat them alike
          CHECK(sc.lo == lo && sc.hi == hi, "scan %s case %d: lo %g/%g hi %g/%g", w.name, c,
                sc.lo, lo, sc.hi, hi);
        }
        CHECK(std::memcmp(oid.data(), id.data(), 4ull * K) == 0 &&
                  std::memcmp(olp.data(), lp.data(), 4ull * K) == 0,
              "scan %s case %d: copy", w.name, c);
        ++scanned;
      }
    }
  }
  std::printf("%d batches packed, %d rejected, %d streamed batches compared, %d rows scanned, "
              "%d failures\n",
              cases, rejected, streamed, scanned, fails);
  return fails ? 1 : 0;
}

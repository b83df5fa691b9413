// Randomised check of the host-only planners of libkvc (kvc_decode_plan,
// kvc_prefill_plan), built with AddressSanitizer / UndefinedBehaviorSanitizer
// on the host side by tests/test_plan_fuzz_asan.py.  Every plan of a valid
// batch must succeed after at most one capacity retry and satisfy the
// invariants the kernels rely on:
//   decode, segment mode: segments tile the flattened page list in order,
//     each within one page of the others and at most 128 pages; pieces tile
//     every request's pages exactly once, partial indices 0..n-1 (or -1 for a
//     single piece); workspace sized for max_partitions;
//   decode, small-batch mode: one segment and one piece per request, at most
//     16 pages each, no partials;
//   prefill: every query of every request in exactly one work unit per KV
//     head; the workgroup table covers the units once, no workgroup empty,
//     and within each XCD's workgroups the loads (key tiles + 2 per unit)
//     differ by at most one unit's cost.
// Prints "ok <iterations>" and exits 0, or the first violation and exits 1.
#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

#include "kvc.h"

namespace {

int fail(const char* what, int it) {
  std::printf("violation at iteration %d: %s (%s)\n", it, what, kvc_last_error());
  return 1;
}

#define CHECK(cond, what) \
  do {                    \
    if (!(cond)) return fail(what, it); \
  } while (0)

int check_decode(const std::vector<int32_t>& indptr, const std::vector<int32_t>& lpl,
                 const kvc_decode_schedule& s, const std::vector<int32_t>& img, int it) {
  const int B = s.batch;
  const int64_t total = B ? indptr[B] : 0;
  CHECK(s.total_pages == total, "total_pages");
  CHECK(s.plan_ints == kvc_decode_plan_ints(B, s.num_segments), "plan_ints");
  const int32_t* seg = img.data();
  const int32_t* pc = img.data() + s.pieces_offset;
  const int32_t* np = img.data() + s.nparts_offset;
  CHECK(int64_t(s.nparts_offset) + B <= int64_t(img.size()), "nparts inside the image");
  if (s.small_batch) {
    CHECK(s.num_segments == B && s.num_pieces == B && s.max_partitions == 1, "small shape");
    CHECK(s.workspace_bytes == 0 && s.heads_per_group == 1, "small workspace");
    for (int b = 0; b < B; ++b) {
      CHECK(indptr[b + 1] - indptr[b] <= 16, "small request within 16 pages");
      CHECK(pc[8 * b] == b && pc[8 * b + 1] == indptr[b] && pc[8 * b + 2] == indptr[b + 1],
            "small piece = request");
      CHECK(pc[8 * b + 3] == -1 && pc[8 * b + 4] == indptr[b + 1] - 1 &&
                pc[8 * b + 5] == lpl[b], "small piece tail");
      CHECK(np[b] == (indptr[b + 1] > indptr[b] ? 1 : 0), "small nparts");
    }
    return 0;
  }
  const int S = s.num_segments;
  CHECK((total == 0) == (S == 0), "segments iff pages");
  std::vector<int> seen(B, 0);
  int64_t min_len = INT64_MAX, max_len = 0;
  int max_parts = 1;
  for (int i = 0; i < S; ++i) {
    const int32_t* r = seg + 4 * i;
    CHECK(r[0] <= r[1] && r[1] <= s.num_pieces, "segment piece range");
    CHECK(i == 0 || r[0] == seg[4 * (i - 1) + 1], "segments contiguous in pieces");
    CHECK(r[2] == (i == 0 ? 0 : seg[4 * (i - 1) + 2] + seg[4 * (i - 1) + 3]), "segments contiguous in slots");
    CHECK(r[3] >= 1 && (i + 1 < S || r[2] + r[3] == total), "segment pages");
    min_len = std::min<int64_t>(min_len, r[3]);
    max_len = std::max<int64_t>(max_len, r[3]);
    int64_t slot = r[2];
    for (int k = r[0]; k < r[1]; ++k) {
      const int32_t* p = pc + 8 * k;
      CHECK(p[0] >= 0 && p[0] < B, "piece request");
      CHECK(p[1] == slot && p[2] > p[1], "pieces contiguous and non-empty");
      CHECK(p[1] >= indptr[p[0]] && p[2] <= indptr[p[0] + 1], "piece inside its request");
      CHECK(p[4] == indptr[p[0] + 1] - 1 && p[5] == lpl[p[0]], "piece tail");
      slot = p[2];
      ++seen[p[0]];
    }
    CHECK(slot == r[2] + r[3], "segment fully covered");
  }
  if (S) CHECK(min_len >= 1 && max_len <= 128, "segments within 1..128 pages");
  for (int b = 0; b < B; ++b) {
    CHECK(seen[b] == np[b], "nparts");
    CHECK((indptr[b + 1] == indptr[b]) == (np[b] == 0), "empty requests have no piece");
    max_parts = std::max(max_parts, np[b]);
  }
  CHECK(s.max_partitions == max_parts, "max_partitions");
  CHECK(s.workspace_bytes ==
            kvc_decode_workspace_bytes(B, s.num_qo_heads, s.head_dim, s.max_partitions),
        "workspace bytes");
  return 0;
}

int check_prefill(const std::vector<int32_t>& qo, const std::vector<int32_t>& kv, int hkv,
                  const kvc_prefill_schedule& s, const std::vector<int32_t>& img, int it) {
  const int B = s.batch;
  const int64_t units = int64_t(s.num_items) * hkv;
  const int64_t W = std::min<int64_t>(256, units);
  const int64_t table = (2 * W + 3) / 4 * 4;
  CHECK(s.plan_ints == table + 8 * units, "prefill plan_ints");
  // the workgroup table covers the unit records once, in order, none empty
  int64_t next = 0;
  std::vector<int64_t> load(W, 0);
  int64_t max_cost = 0;
  for (int64_t w = 0; w < W; ++w) {
    CHECK(img[2 * w] == next && img[2 * w + 1] >= 1, "workgroup table");
    for (int64_t u = next; u < next + img[2 * w + 1]; ++u) {
      const int64_t c = img[table + 8 * u + 6] + 2;
      load[w] += c;
      max_cost = std::max(max_cost, c);
    }
    next += img[2 * w + 1];
  }
  CHECK(next == units, "every unit in one workgroup");
  // list scheduling: within each XCD's workgroups, loads within one unit's cost
  const int groups = W % 8 == 0 ? 8 : 1;
  for (int x = 0; x < groups; ++x) {
    int64_t lo = INT64_MAX, hi = 0;
    for (int64_t w = x; w < W; w += groups) lo = std::min(lo, load[w]), hi = std::max(hi, load[w]);
    CHECK(hi - lo <= max_cost, "workgroup balance");
  }
  // every query of every request in exactly one unit per KV head
  std::vector<int> req_of_q(qo.empty() ? 0 : size_t(qo[B]) + 1, -1);
  for (int b = 0; b < B; ++b)
    if (qo[b + 1] > qo[b]) req_of_q[size_t(qo[b])] = b;
  std::vector<int64_t> covered(size_t(B) * hkv, 0);
  for (int64_t u = 0; u < units; ++u) {
    const int32_t* r = img.data() + table + 8 * u;
    CHECK(r[0] >= 0 && r[0] < hkv, "unit head");
    CHECK(r[4] >= 0 && r[4] < int64_t(req_of_q.size()) && req_of_q[size_t(r[4])] >= 0,
          "unit request");
    const int b = req_of_q[size_t(r[4])];
    CHECK(r[2] == qo[b + 1] - qo[b] && r[5] == kv[b], "unit offsets");
    CHECK(r[1] >= 0 && r[1] < r[2] && r[1] % s.tile_tokens == 0, "unit first query");
    covered[size_t(b) * hkv + r[0]] += std::min(r[1] + s.tile_tokens, r[2]) - r[1];
  }
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < hkv; ++h)
      CHECK(covered[size_t(b) * hkv + h] == qo[b + 1] - qo[b], "queries covered once per head");
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  const int iters = argc > 1 ? std::atoi(argv[1]) : 2000;
  std::mt19937 rng(20261202);
  const int dims[3] = {64, 128, 256};
  for (int it = 0; it < iters; ++it) {
    const int B = int(rng() % 300);
    const bool short_ctx = rng() % 3 == 0;
    std::vector<int32_t> indptr(B + 1, 0), lpl(B, 0);
    for (int b = 0; b < B; ++b) {
      const int len = rng() % 5 == 0 ? 0
                      : short_ctx    ? int(rng() % 300)
                                     : int(rng() % (rng() % 4 == 0 ? 40000 : 3000));
      indptr[b + 1] = indptr[b] + (len + 15) / 16;
      lpl[b] = len == 0 ? 0 : (len % 16 ? len % 16 : 16);
    }
    const int hkv = 1 << (rng() % 5), g = 1 << (rng() % 4);
    const int d = dims[rng() % 3];
    const int hint = rng() % 4 == 0 ? int(rng() % 2000) : 0;
    const int cus = int(rng() % 300) + 1;
    kvc_decode_schedule s{};
    std::vector<int32_t> img(size_t(rng() % 64 + 1));
    int st = kvc_decode_plan(indptr.data(), lpl.data(), B, hkv * g, hkv, d, 16, hint, cus, &s,
                             img.data(), int64_t(img.size()));
    if (st == KVC_ERR_WORKSPACE) {
      CHECK(s.plan_ints > int64_t(img.size()), "capacity report");
      img.assign(size_t(s.plan_ints), -7);
      st = kvc_decode_plan(indptr.data(), lpl.data(), B, hkv * g, hkv, d, 16, hint, cus, &s,
                           img.data(), int64_t(img.size()));
    }
    CHECK(st == KVC_OK, "decode plan of a valid batch");
    if (check_decode(indptr, lpl, s, img, it)) return 1;

    // Prefill: chunks of at most each request's cached tokens.
    std::vector<int32_t> qo(B + 1, 0);
    for (int b = 0; b < B; ++b) {
      const int len = (indptr[b + 1] - indptr[b]) * 16 - (lpl[b] ? 16 - lpl[b] : 0);
      qo[b + 1] = qo[b] + (len ? int(rng() % (len + 1)) : 0);
    }
    kvc_prefill_schedule ps{};
    std::vector<int32_t> pimg(size_t(rng() % 256 + 1));
    const int causal = int(rng() % 2);
    st = kvc_prefill_plan(qo.data(), indptr.data(), lpl.data(), B, hkv * g, hkv, 128, 16,
                          causal, &ps, pimg.data(), int64_t(pimg.size()));
    if (st == KVC_ERR_WORKSPACE) {
      CHECK(ps.plan_ints > int64_t(pimg.size()), "prefill capacity report");
      pimg.assign(size_t(ps.plan_ints), -7);
      st = kvc_prefill_plan(qo.data(), indptr.data(), lpl.data(), B, hkv * g, hkv, 128, 16,
                            causal, &ps, pimg.data(), int64_t(pimg.size()));
    }
    CHECK(st == KVC_OK, "prefill plan of a valid batch");
    if (check_prefill(qo, indptr, hkv, ps, pimg, it)) return 1;
  }
  std::printf("ok %d\n", iters);
  return 0;
}

// Segment planner (host code, no GPU access): the segment table that the chunked
// prefills (hmx_gdn_chunk_fwd, hmx_gka_chunk_fwd, hmx_ssd_chunk_fwd) take.
//
// A prefill runs one workgroup per (segment, head).  Every sequence is cut into
// chunk-aligned segments so that the GPU is filled whatever the batch: one long
// sequence is split into many segments, a batch of many short ones keeps one
// segment each.  Segment counts are handed out one at a time to the sequence
// whose segments are currently the longest (the longest segment bounds the
// runtime when all of them run at once), down to kMinSegmentChunks chunks per
// segment, for a budget of one or two waves of concurrent workgroups; the budget
// with the smaller estimated makespan wins (the longest segment plus the
// kWarmChunks of start-state recomputation a split sequence pays, times the waves).
#include <algorithm>
#include <climits>
#include <queue>
#include <vector>

#include "common.hpp"

namespace hmx {
namespace plan {

struct OpShape { int chunk; int wg_per_cu; };
// GDN walks 32-token chunks, GKA 64-token blocks, SSD 64-token chunks; each runs
// two workgroups per CU
constexpr OpShape kOps[] = {{32, 2}, {64, 2}, {64, 2}};
constexpr int kMinSegmentChunks = 16;
constexpr int kWarmChunks = 3;

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

std::vector<int64_t> balanced_counts(const std::vector<int64_t>& chunks, int64_t budget) {
  std::vector<int64_t> ns(chunks.size(), 1);
  // pop order: the longest current segment first, the lower sequence index on ties
  struct Item { double len; int64_t n; };
  auto later = [](const Item& a, const Item& b) { return a.len < b.len || (a.len == b.len && a.n > b.n); };
  std::priority_queue<Item, std::vector<Item>, decltype(later)> heap(later);
  for (size_t n = 0; n < chunks.size(); ++n) heap.push(Item{(double)chunks[n], (int64_t)n});
  int64_t total = (int64_t)chunks.size();
  while (total < budget && !heap.empty()) {
    const Item it = heap.top();
    heap.pop();
    const int64_t n = it.n;
    if (it.len < 2.0 * kMinSegmentChunks ||
        (double)chunks[n] / (double)(ns[n] + 1) < (double)kMinSegmentChunks)
      continue;  // too short to split further
    ns[n] += 1;
    total += 1;
    heap.push(Item{(double)chunks[n] / (double)ns[n], n});
  }
  return ns;
}

int build(int op, const int64_t* bos_eos, int nseq, int64_t tokens, int H, int cu_count,
          int segment_chunks, int32_t* table, int max_rows, int32_t* nrows, int32_t* nblock_total) {
  HMX_REQUIRE(op >= 0 && op < (int)(sizeof(kOps) / sizeof(kOps[0])), HMX_EINVAL,
              "hmx_plan_segments: unknown op %d", op);
  HMX_REQUIRE(nseq >= 0 && H > 0 && cu_count > 0 && segment_chunks >= 0, HMX_EINVAL,
              "hmx_plan_segments: bad sizes (nseq %d, H %d, cu_count %d, segment_chunks %d)",
              nseq, H, cu_count, segment_chunks);
  HMX_REQUIRE(nseq == 0 || bos_eos, HMX_EINVAL, "hmx_plan_segments: NULL sequence bounds");
  HMX_REQUIRE(nrows, HMX_EINVAL, "hmx_plan_segments: NULL nrows");
  for (int n = 0; n < nseq; ++n) {
    const int64_t b = bos_eos[2 * n], e = bos_eos[2 * n + 1];
    HMX_REQUIRE(0 <= b && b <= e && e <= tokens, HMX_EINVAL,
                "hmx_plan_segments: sequence %d spans [%lld, %lld), outside [0, %lld]", n,
                (long long)b, (long long)e, (long long)tokens);
  }
  const int chunk = kOps[op].chunk;
  std::vector<int64_t> chunks(nseq), counts;
  for (int n = 0; n < nseq; ++n) chunks[n] = ceil_div(bos_eos[2 * n + 1] - bos_eos[2 * n], chunk);
  if (segment_chunks > 0) {
    counts.resize(nseq);
    for (int n = 0; n < nseq; ++n) counts[n] = std::max<int64_t>(1, ceil_div(chunks[n], segment_chunks));
  } else {
    const int64_t slots = std::max<int64_t>(1, (int64_t)kOps[op].wg_per_cu * cu_count / H);
    int64_t best_est = -1;
    for (int waves = 1; waves <= 2; ++waves) {
      std::vector<int64_t> cnt = balanced_counts(chunks, waves * slots);
      int64_t longest = 0, sum = 0;
      for (int n = 0; n < nseq; ++n) {
        longest = std::max(longest, ceil_div(chunks[n], cnt[n]) + (cnt[n] > 1 ? kWarmChunks : 0));
        sum += cnt[n];
      }
      // segments beyond one wave of slots queue behind the first wave
      const int64_t est = longest * std::min<int64_t>(waves, ceil_div(sum, slots));
      if (best_est < 0 || est < best_est) {
        best_est = est;
        counts = std::move(cnt);
      }
    }
  }
  int64_t rows = 0, blocks = 0;
  for (int n = 0; n < nseq; ++n) rows += counts[n];
  HMX_REQUIRE(rows <= INT32_MAX / 8, HMX_EINVAL, "hmx_plan_segments: %lld segments", (long long)rows);
  *nrows = (int32_t)rows;
  for (int n = 0; n < nseq; ++n) blocks += chunks[n];
  if (nblock_total) *nblock_total = (int32_t)blocks;
  if (!table) return HMX_OK;
  HMX_REQUIRE(max_rows >= rows, HMX_EINVAL, "hmx_plan_segments: the table needs %lld rows, has %d",
              (long long)rows, max_rows);
  int32_t* r = table;
  for (int n = 0; n < nseq; ++n) {
    const int64_t first = r - table, nc = chunks[n], ns = counts[n];
    for (int64_t i = 0; i < ns; ++i, r += 8) {
      r[0] = n;
      r[1] = (int32_t)bos_eos[2 * n];
      r[2] = (int32_t)bos_eos[2 * n + 1];
      r[3] = (int32_t)(i * nc / ns);
      r[4] = (int32_t)((i + 1) * nc / ns);
      r[5] = (int32_t)i;
      r[6] = (int32_t)(first / 8);
      r[7] = (int32_t)ns;
    }
  }
  return HMX_OK;
}

}  // namespace plan
}  // namespace hmx

extern "C" int hmx_plan_segments_bounds(int32_t op, const int64_t* bos_eos, int32_t nseq,
                                        int64_t tokens, int32_t H, int32_t cu_count,
                                        int32_t segment_chunks, int32_t* table, int32_t max_rows,
                                        int32_t* nrows, int32_t* nblock_total) {
  return hmx::plan::build(op, bos_eos, nseq, tokens, H, cu_count, segment_chunks, table, max_rows,
                          nrows, nblock_total);
}

extern "C" int hmx_plan_segments(int32_t op, const int64_t* cu_seqlens, int32_t nseq, int32_t B,
                                 int64_t T, int32_t H, int32_t cu_count, int32_t segment_chunks,
                                 int32_t* table, int32_t max_rows, int32_t* nrows,
                                 int32_t* nblock_total) {
  HMX_REQUIRE(B >= 0 && T >= 0, HMX_EINVAL, "hmx_plan_segments: bad B %d / T %lld", B, (long long)T);
  std::vector<int64_t> be;
  if (!cu_seqlens) {
    HMX_REQUIRE(nseq == B, HMX_EINVAL, "hmx_plan_segments: without cu_seqlens nseq must be B");
    for (int n = 0; n < B; ++n) {
      be.push_back((int64_t)n * T);
      be.push_back((int64_t)n * T + T);
    }
  } else {
    HMX_REQUIRE(nseq >= 0 && cu_seqlens[0] == 0, HMX_EINVAL,
                "hmx_plan_segments: cu_seqlens must start at 0");
    for (int n = 0; n < nseq; ++n) {
      HMX_REQUIRE(cu_seqlens[n + 1] >= cu_seqlens[n], HMX_EINVAL,
                  "hmx_plan_segments: cu_seqlens decreases at %d", n);
      be.push_back(cu_seqlens[n]);
      be.push_back(cu_seqlens[n + 1]);
    }
  }
  return hmx::plan::build(op, be.data(), nseq, (int64_t)B * T, H, cu_count, segment_chunks, table,
                          max_rows, nrows, nblock_total);
}

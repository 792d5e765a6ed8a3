// The attention kernel's persistent schedule, built on the host from a plan's
// row lengths. Pure C++, no device code: h3hip_plan_create uploads the result,
// and h3hip_schedule exposes the same lists to callers and tests.
#include <algorithm>
#include <cstdint>
#include <numeric>
#include <queue>
#include <vector>

#include "plan.h"

namespace h3hip {

// The attention kernel's schedule: which (head, q-tile) work units each of
// its persistent workgroups runs, and in what order.
//
// Workgroups are handed to the 8 XCDs round-robin (workgroup b runs on XCD
// b % 8), and each XCD has its own L2. So each XCD gets its own list, laid
// out for L2 reuse: long rows (the dense prefix rows, ~8x the median) first,
// grouped by head so that units streaming the same head's K/V run side by
// side, then a contiguous (head, q-tile) range so neighbouring q-tiles of one
// head, which share most of their key tiles under local masks, are resident
// together. The XCD lists are balanced by cost (tiles + a fixed per-unit
// overhead). Each list is then dealt to the XCD's workgroups in list order,
// every unit to the workgroup that the cost model frees first -- the order in
// which the hardware's own dispatch would hand them out -- so the units an
// XCD runs at one time stay neighbours in its list.
// Cost of a unit in tile times beyond its tiles (merge, store, first loads),
// measured on MI355X (band rules: 1.8 us per tile, the rest per unit).
constexpr double kUnitOverhead = 2.0;

int build_schedule(const std::vector<int32_t>& row_ptr, int32_t heads, int32_t groups,
                   std::vector<int32_t>& work_ptr, std::vector<int32_t>& work) {
  const int32_t nq = (int32_t)row_ptr.size() - 1;
  const int kXcd = 8;
  std::vector<int32_t> len(nq);
  for (int32_t i = 0; i < nq; i++) len[i] = row_ptr[i + 1] - row_ptr[i];
  std::vector<int32_t> sorted_len(len);
  std::sort(sorted_len.begin(), sorted_len.end());
  const int32_t median = nq ? sorted_len[nq / 2] : 0;
  const int32_t long_at = std::max<int32_t>(4 * median, median + 16);

  std::vector<std::vector<int32_t>> lists(kXcd);
  std::vector<double> cost(kXcd, 0.0);
  auto enc = [](int32_t h, int32_t qt) { return (h << 16) | qt; };

  // Long rows, one group per head, groups placed greedily on the least-loaded XCD.
  std::vector<int32_t> long_rows;
  for (int32_t i = 0; i < nq; i++)
    if (len[i] >= long_at) long_rows.push_back(i);
  std::stable_sort(long_rows.begin(), long_rows.end(),
                   [&](int32_t a, int32_t b) { return len[a] > len[b]; });
  double long_cost = 0;
  for (int32_t i : long_rows) long_cost += len[i] + kUnitOverhead;
  for (int32_t h = 0; h < heads && !long_rows.empty(); h++) {
    const int x = (int)(std::min_element(cost.begin(), cost.end()) - cost.begin());
    for (int32_t i : long_rows) lists[x].push_back(enc(h, i));
    cost[x] += long_cost;
  }

  // Regular rows: one contiguous (head, q-tile) sequence split into ranges that
  // top every XCD up to the same total.
  std::vector<int32_t> regular;
  double reg_cost = 0;
  for (int32_t h = 0; h < heads; h++)
    for (int32_t i = 0; i < nq; i++)
      if (len[i] < long_at) {
        regular.push_back(enc(h, i));
        reg_cost += len[i] + kUnitOverhead;
      }
  double total = reg_cost;
  for (double c : cost) total += c;
  const double target = total / kXcd;
  size_t pos = 0;
  // Fill the least-loaded XCDs first so ranges stay contiguous per XCD.
  std::vector<int> order(kXcd);
  std::iota(order.begin(), order.end(), 0);
  std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return cost[a] < cost[b]; });
  for (int oi = 0; oi < kXcd; oi++) {
    const int x = order[oi];
    while (pos < regular.size() && (oi == kXcd - 1 || cost[x] < target)) {
      const int32_t qt = regular[pos] & 0xffff;
      lists[x].push_back(regular[pos]);
      cost[x] += len[qt] + kUnitOverhead;
      pos++;
    }
  }
  // Each XCD's list onto its groups / 8 workgroups (workgroup c*8 + x is the
  // c-th of XCD x).
  const int per_xcd = groups / kXcd;
  std::vector<std::vector<int32_t>> per_wg(groups);
  for (int x = 0; x < kXcd; x++) {
    std::priority_queue<std::pair<double, int>, std::vector<std::pair<double, int>>,
                        std::greater<std::pair<double, int>>>
        free_at;
    for (int c = 0; c < per_xcd; c++) free_at.push({0.0, c});
    for (int32_t u : lists[x]) {
      const auto [t, c] = free_at.top();
      free_at.pop();
      per_wg[c * kXcd + x].push_back(u);
      free_at.push({t + len[u & 0xffff] + kUnitOverhead, c});
    }
  }
  work_ptr.assign(groups + 1, 0);
  work.clear();
  for (int b = 0; b < groups; b++) {
    work.insert(work.end(), per_wg[b].begin(), per_wg[b].end());
    work_ptr[b + 1] = (int32_t)work.size();
  }
  // Every (head, q-tile) unit exactly once: a dropped unit would leave its
  // output rows unwritten, a duplicated one would race with itself.
  std::vector<uint8_t> seen((size_t)heads * nq, 0);
  bool ok = work.size() == (size_t)heads * nq;
  for (size_t i = 0; ok && i < work.size(); i++) {
    const int32_t h = work[i] >> 16, qt = work[i] & 0xffff;
    ok = h >= 0 && h < heads && qt < nq && !seen[(size_t)h * nq + qt];
    if (ok) seen[(size_t)h * nq + qt] = 1;
  }
  if (!ok) {
    set_error("internal: the attention schedule does not list each of the %lld units once",
              (long long)heads * nq);
    return H3HIP_EHIP;
  }
  return H3HIP_OK;
}


}  // namespace h3hip

extern "C" int h3hip_schedule(const int32_t* row_ptr, int32_t n_tiles, int32_t heads,
                              int32_t groups, int32_t* work_ptr, int32_t* work) {
  using h3hip::set_error;
  if (!row_ptr || !work_ptr || !work) {
    set_error("NULL argument");
    return H3HIP_EINVAL;
  }
  if (n_tiles <= 0 || n_tiles > 32767 || heads <= 0 || heads >= 32768 || groups <= 0 ||
      groups % 8 != 0) {
    set_error("bad shape: n_tiles %d heads %d groups %d (groups a positive multiple of 8)",
              n_tiles, heads, groups);
    return H3HIP_EINVAL;
  }
  std::vector<int32_t> rp(row_ptr, row_ptr + n_tiles + 1);
  if (rp[0] != 0) {
    set_error("row_ptr[0] must be 0");
    return H3HIP_EINVAL;
  }
  for (int32_t i = 0; i < n_tiles; i++)
    if (rp[i + 1] < rp[i] || rp[i + 1] - rp[i] > n_tiles) {
      set_error("row_ptr is not a CSR row pointer over %d columns at row %d", n_tiles, i);
      return H3HIP_EINVAL;
    }
  std::vector<int32_t> wp, w;
  const int rc = h3hip::build_schedule(rp, heads, groups, wp, w);
  if (rc != H3HIP_OK) return rc;
  std::copy(wp.begin(), wp.end(), work_ptr);
  std::copy(w.begin(), w.end(), work);
  return H3HIP_OK;
}

// The opaque plan behind h3hip_plan: tile lists (host and device), launch
// order and decline policy. Immutable after h3hip_plan_create.
#pragma once

#include <cstdint>
#include <vector>

#include "../../include/ch3hip.h"

struct h3hip_plan_s {
  int32_t seq_len = 0;
  int32_t seq_pad = 0;
  int32_t n_tiles = 0;
  int32_t heads = 0;
  int32_t prefix_len = 0;
  int32_t kind = 0;
  int64_t nnz = 0;
  h3hip_policy policy{};
  std::vector<int32_t> row_ptr;  // host copy [n_tiles + 1]
  std::vector<int32_t> col_idx;  // host copy [nnz]
  // Attention schedule: one persistent workgroup per CU; workgroup b (on XCD
  // b % 8) runs the units work[work_ptr[b] .. work_ptr[b + 1]), each
  // (head << 16 | q_tile), in order.
  int32_t groups = 0;
  std::vector<int32_t> work_ptr;  // [groups + 1]
  std::vector<int32_t> work;
  int32_t* d_row_ptr = nullptr;
  int32_t* d_col_idx = nullptr;
  int32_t* d_work_ptr = nullptr;
  int32_t* d_work = nullptr;
  // One descriptor per unit, in work order, kUnitDescInts int32 each: what
  // the attention kernel needs at a unit's start, in one scalar load instead
  // of a chain of dependent ones (unit -> row_ptr -> col_idx).
  std::vector<int32_t> unit_desc;
  int32_t* d_unit_desc = nullptr;
};

// Unit descriptor layout: unit (head << 16 | q_tile), first index of the row
// in col_idx, tile count n, columns c0, c1, c2 (the first three, repeating the
// last when n < 3), ragged (1 when the last tile runs past seq_len), unused.
constexpr int kUnitDescInts = 8;

namespace h3hip {

// Thread-local last error (defined with the plan code); the ABI is re-entrant
// per thread.
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

// The persistent attention schedule for these CSR rows (schedule.cpp):
// work_ptr[groups + 1] and work[heads * n_tiles], each unit (head << 16 |
// q_tile) listed once. H3HIP_OK, or an error with the message set.
int build_schedule(const std::vector<int32_t>& row_ptr, int32_t heads, int32_t groups,
                   std::vector<int32_t>& work_ptr, std::vector<int32_t>& work);

}  // namespace h3hip

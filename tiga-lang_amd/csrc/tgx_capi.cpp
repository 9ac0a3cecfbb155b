// Host-only parts of the C ABI: status strings, per-thread error message and
// the restatement of the reference's degree-bucket planner decisions.
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include <algorithm>
#include <vector>

#include "tgx.h"

namespace tgx {

static thread_local char g_last_error[1024] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

}  // namespace tgx

extern "C" const char* tgx_status_string(int status) {
  switch (status) {
    case TGX_OK: return "ok";
    case TGX_INVALID_ARGUMENT: return "invalid argument";
    case TGX_UNSUPPORTED: return "unsupported";
    case TGX_OUT_OF_MEMORY: return "out of memory";
    case TGX_INTERNAL: return "internal error";
    default: return "unknown status";
  }
}

extern "C" const char* tgx_last_error(void) { return tgx::g_last_error; }

extern "C" int tgx_abi_version(void) { return 13; }

// ---------------------------------------------------------------------------
// Reference planner restatement.
//
//   annotateLoadBalance   lib/Transforms/SelectKernelSchedule.cpp:136-163
//   makeUpperBounds       lib/Transforms/PlanDegreeBuckets.cpp:32-44
//   bucket planning       lib/Transforms/PlanDegreeBuckets.cpp:86-143, 221-261
//   split-row planning    lib/Transforms/PlanSplitRows.cpp:84-147
//
// The reference runs these as MLIR passes over a launch op; here the same
// decisions are a pure function of (rows, max degree, degree sum, optional
// exact histogram, node epilogue present).  The MI355X kernels use their own
// row bins; this planner exists so the reference's schedule decisions can be
// reported by explain() and checked against the reference's lit vectors.
namespace {

enum PlanCode {
  kRowNeighborTile = 0,
  kDegreeBucketing = 1,
  kTailSplit = 2,
  kDeferredHighDegree = 3,
  kBoundedRowPreferred = 4,
  kTailChunked = 5,
  kTailRowSplit = 6,
};

int64_t next_pow2(int64_t v) {
  int64_t p = 1;
  while (p < v) p <<= 1;
  return p;
}

std::vector<int64_t> upper_bounds(int64_t maximum) {
  std::vector<int64_t> b;
  int64_t bound = 8;
  while (bound < maximum) {
    b.push_back(bound);
    if (bound > INT64_MAX / 2) break;
    bound *= 2;
  }
  if (b.empty() || b.back() != maximum) b.push_back(maximum);
  return b;
}

}  // namespace

extern "C" int tgx_plan_reference_buckets(
    int64_t n_rows, int64_t max_degree, int64_t degree_sum, const int64_t* histogram,
    int has_node_epilogue, int* plan_code, int64_t* utilization_milli,
    int64_t* bounds_out, int* mapping_out, int64_t* rows_in_bucket_out, int* n_bounds,
    int64_t* partials_per_row, int64_t* active_rows) {
  if (!plan_code || !utilization_milli || !bounds_out || !mapping_out ||
      !rows_in_bucket_out || !n_bounds || !partials_per_row || !active_rows) {
    tgx::set_error("null output pointer");
    return TGX_INVALID_ARGUMENT;
  }
  *utilization_milli = -1;
  *n_bounds = 0;
  *partials_per_row = 0;
  *active_rows = 0;
  if (n_rows <= 0 || max_degree <= 0) {
    *plan_code = kRowNeighborTile;
    return TGX_OK;
  }
  // annotateLoadBalance
  bool bucketing;
  if (max_degree > 64) {
    bucketing = true;
  } else {
    const int64_t padded = next_pow2(max_degree);
    const long double util = 1000.0L * static_cast<long double>(degree_sum) /
                             (static_cast<long double>(n_rows) * padded);
    *utilization_milli = static_cast<int64_t>(util);
    bucketing = *utilization_milli < 600;
  }
  if (!bucketing) {
    *plan_code = kRowNeighborTile;
    return TGX_OK;
  }
  // PlanDegreeBuckets
  if (!histogram && max_degree > 64) {
    *plan_code = kDeferredHighDegree;
    return TGX_OK;
  }
  std::vector<int64_t> bounds = upper_bounds(max_degree);
  bool tail_split = false;
  int code = kDegreeBucketing;
  if (histogram && max_degree > 32) {
    const int64_t threshold = max_degree > 64 ? 64 : max_degree / 2;
    int64_t tail_rows = 0;
    for (int64_t d = threshold + 1; d <= max_degree; ++d) tail_rows += histogram[d];
    if (max_degree > 64 || tail_rows * 10 <= n_rows) {
      int64_t short_bound = threshold;
      if (max_degree > 64) {
        int64_t cumulative = 0, previous = -1;
        for (int64_t candidate : {8, 16, 32}) {
          for (int64_t d = previous + 1; d <= candidate; ++d) cumulative += histogram[d];
          previous = candidate;
          if (cumulative * 2 >= n_rows) {
            short_bound = candidate;
            break;
          }
        }
      }
      if (short_bound < threshold && !has_node_epilogue)
        bounds = {short_bound, max_degree};
      else if (short_bound < threshold)
        bounds = {short_bound, threshold, max_degree};
      else
        bounds = {threshold, max_degree};
      tail_split = true;
      code = kTailSplit;
    }
  }
  if (histogram && max_degree <= 32) {
    *plan_code = kBoundedRowPreferred;
    return TGX_OK;
  }
  if (bounds.size() > 64) {
    tgx::set_error("too many buckets");
    return TGX_INTERNAL;
  }
  int64_t lower = -1;
  for (size_t k = 0; k < bounds.size(); ++k) {
    int64_t rows_in = n_rows;
    if (histogram) {
      rows_in = 0;
      for (int64_t d = lower + 1; d <= bounds[k]; ++d) rows_in += histogram[d];
    }
    bounds_out[k] = bounds[k];
    mapping_out[k] = (tail_split && k == 0) ? 1 : 0;
    rows_in_bucket_out[k] = rows_in;
    lower = bounds[k];
  }
  *n_bounds = static_cast<int>(bounds.size());
  // PlanSplitRows: only after a tail split with max > 64 and a bucket that
  // starts in (0, 64] and ends at max with worklist mapping.
  if (tail_split && max_degree > 64) {
    int tail = -1;
    lower = -1;
    for (int k = 0; k < *n_bounds; ++k) {
      if (lower > 0 && lower <= 64 && bounds_out[k] == max_degree && mapping_out[k] == 0) {
        tail = k;
        break;
      }
      lower = bounds_out[k];
    }
    if (tail >= 0 && rows_in_bucket_out[tail] > 0) {
      if (!has_node_epilogue) {
        mapping_out[tail] = 2;
        code = kTailChunked;
      } else {
        *partials_per_row = (max_degree + 63) / 64;
        *active_rows = rows_in_bucket_out[tail];
        code = kTailRowSplit;
      }
    }
  }
  *plan_code = code;
  return TGX_OK;
}

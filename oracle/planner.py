"""Reference degree-bucket planner decisions (pure Python restatement).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Restates, as one pure function of (rows, max degree, degree sum, exact
histogram or None, node epilogue present):
  annotateLoadBalance   lib/Transforms/SelectKernelSchedule.cpp:136-163
  makeUpperBounds       lib/Transforms/PlanDegreeBuckets.cpp:32-44
  bucket planning       lib/Transforms/PlanDegreeBuckets.cpp:86-143, 221-261
  split-row planning    lib/Transforms/PlanSplitRows.cpp:84-147 (single
                        associative f32 reducer)
Pinned by the reference's lit vectors (tests/mlir/plan-degree-buckets.mlir,
power-law-cdf-split.mlir, plan-split-rows.mlir, tail-split-to-bundle.mlir,
kernel-load-balance-analysis.mlir, plan-degree-buckets-deferred.mlir),
restated as data in tests/golden/reference_vectors.json.
"""

from __future__ import annotations

PLAN_NAMES = {
    0: "row-neighbor-tile",
    1: "degree-bucketing-required",
    2: "high-degree-tail-split",
    3: "provider-deferred-high-degree",
    4: "bounded-row-preferred",
    5: "high-degree-tail-chunked",
    6: "high-degree-tail-split-rows",
}
MAPPING_NAMES = {0: "worklist", 1: "direct-filter", 2: "worklist-chunked"}


def _next_pow2(v):
    p = 1
    while p < v:
        p <<= 1
    return p


def upper_bounds(maximum):
    bounds = []
    bound = 8
    while bound < maximum:
        bounds.append(bound)
        bound *= 2
    if not bounds or bounds[-1] != maximum:
        bounds.append(maximum)
    return bounds


def plan(rows, max_degree, degree_sum, histogram=None, has_node=False):
    """Return a dict: plan, utilization_milli, bounds, mapping, rows_in_bucket,
    partials_per_row, active_rows."""
    res = {"plan": "row-neighbor-tile", "utilization_milli": -1, "bounds": [],
           "mapping": [], "rows_in_bucket": [], "partials_per_row": 0, "active_rows": 0}
    if rows <= 0 or max_degree <= 0:
        return res
    if max_degree > 64:
        bucketing = True
    else:
        util = int(1000 * degree_sum / (rows * _next_pow2(max_degree)))
        res["utilization_milli"] = util
        bucketing = util < 600
    if not bucketing:
        return res
    if histogram is None and max_degree > 64:
        res["plan"] = "provider-deferred-high-degree"
        return res
    hist = list(histogram) if histogram is not None else None
    bounds = upper_bounds(max_degree)
    tail_split = False
    code = "degree-bucketing-required"
    if hist is not None and max_degree > 32:
        threshold = 64 if max_degree > 64 else max_degree // 2
        tail_rows = sum(hist[threshold + 1:max_degree + 1])
        if max_degree > 64 or tail_rows * 10 <= rows:
            short = threshold
            if max_degree > 64:
                cumulative, previous = 0, -1
                for candidate in (8, 16, 32):
                    cumulative += sum(hist[previous + 1:candidate + 1])
                    previous = candidate
                    if cumulative * 2 >= rows:
                        short = candidate
                        break
            if short < threshold and not has_node:
                bounds = [short, max_degree]
            elif short < threshold:
                bounds = [short, threshold, max_degree]
            else:
                bounds = [threshold, max_degree]
            tail_split = True
            code = "high-degree-tail-split"
    if hist is not None and max_degree <= 32:
        res["plan"] = "bounded-row-preferred"
        return res
    lower = -1
    for k, b in enumerate(bounds):
        res["bounds"].append(b)
        res["mapping"].append("direct-filter" if tail_split and k == 0 else "worklist")
        res["rows_in_bucket"].append(rows if hist is None else sum(hist[lower + 1:b + 1]))
        lower = b
    if tail_split and max_degree > 64:
        lower = -1
        for k, b in enumerate(res["bounds"]):
            if 0 < lower <= 64 and b == max_degree and res["mapping"][k] == "worklist":
                if res["rows_in_bucket"][k] > 0:
                    if not has_node:
                        res["mapping"][k] = "worklist-chunked"
                        code = "high-degree-tail-chunked"
                    else:
                        res["partials_per_row"] = (max_degree + 63) // 64
                        res["active_rows"] = res["rows_in_bucket"][k]
                        code = "high-degree-tail-split-rows"
                break
            lower = b
    res["plan"] = code
    # Bucket launch grid (lib/Target/Triton/Translate.cpp:4728-4830):
    # blockD = nextpow2(upper), blockM = min(16, 256 / blockD),
    # grid_x = ceil((direct-filter ? rows : rows_in_bucket) / blockM).
    grid = []
    for k, b in enumerate(res["bounds"]):
        block_m = max(1, min(16, 256 // _next_pow2(b)))
        count = rows if res["mapping"][k] == "direct-filter" else res["rows_in_bucket"][k]
        grid.append((count + block_m - 1) // block_m)
    res["grid_x"] = grid
    res["worklist_elements"] = rows + 2 * len(res["bounds"]) + 1
    res["partial_bytes"] = 4 * res["partials_per_row"] * res["active_rows"]
    return res

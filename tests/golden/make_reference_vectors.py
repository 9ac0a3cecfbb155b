"""Writes reference_vectors.json: known answers and planner decisions
transcribed from the reference's own tests and examples (each entry cites its
file:line).  Nothing from the reference is imported or executed; the values
are the literals those tests assert.  Run: python tests/golden/make_reference_vectors.py
"""
import json
from pathlib import Path


def hist(pairs, n):
    h = [0] * (n + 1)
    for d, c in pairs.items():
        h[d] = c
    return h


VECTORS = {
    "_source": "Known answers and planner decisions restated as data from the reference's "
               "own tests (file:line per entry). Inputs and expected outputs only.",
    "readme_weighted_sum": {
        "cite": "README.md:91-111; tests/python/test_message_passing_autograd.py:145-180",
        "row_ptr": [0, 2, 3, 5], "col_idx": [0, 2, 1, 0, 1], "num_src": 3,
        "x": [1.0, 2.0, 3.0], "weight": [2.0, 3.0, 4.0, 5.0, 6.0],
        "out": [11.0, 8.0, 17.0], "dx": [7.0, 10.0, 3.0], "dw": [1.0, 3.0, 2.0, 1.0, 2.0]},
    "quickstart_node_bias": {
        "cite": "examples/torch_quickstart.py:16-44",
        "row_ptr": [0, 2, 3, 5], "col_idx": [0, 2, 1, 0, 1], "num_src": 3,
        "x": [1.0, 2.0, 3.0], "weight": [2.0, 3.0, 4.0, 5.0, 6.0], "bias": [0.1, 0.2, 0.3],
        "out": [11.1, 8.2, 17.3], "dx": [7.0, 10.0, 3.0], "dw": [1.0, 3.0, 2.0, 1.0, 2.0],
        "dbias": [1.0, 1.0, 1.0]},
    "online_softmax_large_scores": {
        "cite": "tests/python/test_message_passing_autograd.py:145-149, 318-351 "
                "(src.score, src.value, loss = out.sum())",
        "row_ptr": [0, 2, 3, 5], "col_idx": [0, 2, 1, 0, 1], "num_src": 3,
        "score": [1000.0, 999.0, 998.0], "value": [[1.0, 0.0], [0.0, 2.0], [3.0, 1.0]],
        "out": [[1.2384058, 0.1192029], [0.0, 2.0], [0.7310586, 0.5378829]],
        "dscore": [-0.5115927, 0.1966119, 0.3149807],
        "dvalue": [[1.6118556, 1.6118556], [1.2689414, 1.2689414], [0.1192029, 0.1192029]],
        "places": 5},
    "online_softmax_empty_row_heads": {
        "cite": "tests/python/test_reference.py:416-444 "
                "(row 1 empty -> zeros; compare per-row torch.softmax)",
        "row_ptr": [0, 2, 2, 5], "col_idx": [0, 2, 1, 2, 3], "num_src": 4, "heads": 2, "width": 3,
        "score": [[1000.0, -1000.0], [999.0, -999.0], [0.2, 0.5], [0.7, -0.5], [-0.1, 1.5]]},
    "planner": [
        {"cite": "tests/mlir/kernel-load-balance-analysis.mlir:8-23", "rows": 128, "max": 64,
         "sum": 2048, "histogram": None, "has_node": False,
         "expect": {"plan": "degree-bucketing-required", "utilization_milli": 250}},
        {"cite": "tests/mlir/plan-degree-buckets.mlir:7-25", "rows": 128, "max": 64,
         "sum": 1024, "histogram": None, "has_node": False,
         "expect": {"bounds": [8, 16, 32, 64], "rows_in_bucket": [128, 128, 128, 128],
                    "mapping": ["worklist"] * 4, "worklist_elements": 137}},
        {"cite": "tests/mlir/plan-degree-buckets-deferred.mlir:11-27", "rows": 128, "max": 256,
         "sum": 2048, "histogram": None, "has_node": False,
         "expect": {"plan": "provider-deferred-high-degree"}},
        {"cite": "tests/mlir/power-law-cdf-split.mlir:26-54", "rows": 128, "max": 256,
         "sum": 1664, "histogram": hist({8: 120, 64: 7, 256: 1}, 256), "has_node": False,
         "expect": {"plan": "high-degree-tail-chunked", "bounds": [8, 256],
                    "mapping": ["direct-filter", "worklist-chunked"], "rows_in_bucket": [120, 8]}},
        {"cite": "tests/mlir/plan-split-rows.mlir:20-69", "rows": 128, "max": 256, "sum": 1664,
         "histogram": hist({8: 120, 64: 7, 256: 1}, 256), "has_node": True,
         "expect": {"plan": "high-degree-tail-split-rows", "bounds": [8, 64, 256],
                    "partials_per_row": 4, "active_rows": 1, "partial_bytes": 16}},
        {"cite": "tests/mlir/tail-split-to-bundle.mlir:5-36", "rows": 512, "max": 64,
         "sum": 8000, "histogram": hist({8: 384, 32: 102, 64: 26}, 64), "has_node": False,
         "expect": {"plan": "high-degree-tail-split", "bounds": [32, 64],
                    "mapping": ["direct-filter", "worklist"], "rows_in_bucket": [486, 26],
                    "grid_x": [64, 7]}},
    ],
}

if __name__ == "__main__":
    out = Path(__file__).with_name("reference_vectors.json")
    out.write_text(json.dumps(VECTORS, indent=1))
    print(out)

"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer.

The product's host-only C ABI code (tiga-lang_amd/csrc/tgx_capi.cpp: status
strings, per-thread error messages, the reference planner restatement; and
tiga-lang_amd/csrc/tgx_cpu.cpp: the CPU twins of the device entry points) and
the oracle's C CPU baseline (oracle/cpu_native.c: the threaded forward loop
and the lowered backward) are compiled with g++/gcc and
-fsanitize=address,undefined (host code only; no GPU code is involved) into
a small harness (tests/sanitize/harness.cpp), which then runs the planner on
the lit vectors and on random histograms, the CPU loops on random graphs, and
every CPU twin on random graphs with split hub rows (at 1 and 4 threads,
compared bit for bit) and on broken inputs they must reject.
Any sanitizer report fails the run (halt_on_error, non-zero exit); the
planner and loop results are also checked against the Python oracle (the
twins' values are checked against it in tests/test_cpu_twins.py).
"""

import json
import os
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

from oracle import planner, ref

ROOT = Path(__file__).resolve().parents[1]
GOLD = json.loads((ROOT / "tests" / "golden" / "reference_vectors.json").read_text())
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer",
       "-g", "-O1"]


@pytest.fixture(scope="module")
def harness(tmp_path_factory):
    if not (shutil.which("g++") and shutil.which("gcc")):
        pytest.skip("g++/gcc not available")
    out = tmp_path_factory.mktemp("san")
    obj = out / "cpu_native.o"
    subprocess.run(["gcc", *SAN, "-std=c11", "-c", str(ROOT / "oracle" / "cpu_native.c"),
                    "-o", str(obj)], check=True)
    exe = out / "harness"
    csrc = ROOT / "tiga-lang_amd" / "csrc"
    subprocess.run(["g++", *SAN, "-std=c++17", f"-I{ROOT / 'include'}", f"-I{csrc}",
                    str(ROOT / "tests" / "sanitize" / "harness.cpp"),
                    str(csrc / "tgx_capi.cpp"), str(csrc / "tgx_cpu.cpp"), str(obj),
                    "-pthread", "-o", str(exe)], check=True)
    return exe


def _run(exe, lines):
    # verify_asan_link_order=0: the environment may preload a library of its
    # own ahead of the sanitizer runtime; it is left as it is.
    env = dict(os.environ,
               ASAN_OPTIONS="halt_on_error=1:detect_leaks=1:verify_asan_link_order=0",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    proc = subprocess.run([str(exe)], input="\n".join(lines) + "\n", capture_output=True,
                          text=True, env=env, timeout=300)
    assert proc.returncode == 0, proc.stderr[-4000:]
    assert "runtime error" not in proc.stderr and "Sanitizer" not in proc.stderr, proc.stderr
    return proc.stdout.splitlines()


def _plan_line(rows, mx, total, hist, has_node):
    h = [] if hist is None else list(hist)
    return f"plan {rows} {mx} {total} {int(has_node)} {len(h)} " + " ".join(map(str, h))


def _parse_plan(text):
    t = text.split()
    assert t[0] == "plan", text
    code, util, n = int(t[1]), int(t[2]), int(t[3])
    vals = list(map(int, t[4:]))
    return {"plan": planner.PLAN_NAMES[code], "utilization_milli": util, "bounds": vals[:n],
            "mapping": [planner.MAPPING_NAMES[m] for m in vals[n:2 * n]],
            "rows_in_bucket": vals[2 * n:3 * n], "partials_per_row": vals[3 * n],
            "active_rows": vals[3 * n + 1]}


def test_planner_under_sanitizers(harness):
    cases = [(c["rows"], c["max"], c["sum"], c["histogram"], c["has_node"])
             for c in GOLD["planner"]]
    rng = np.random.default_rng(3)
    for _ in range(300):
        mx = int(rng.integers(1, 600))
        rows = int(rng.integers(1, 800))
        hist = np.zeros(mx + 1, dtype=np.int64)
        np.add.at(hist, rng.integers(0, mx + 1, size=rows), 1)
        hist[mx] += 1
        rows += 1
        total = int((hist * np.arange(mx + 1)).sum())
        cases.append((rows, mx, total, hist.tolist() if rng.random() < 0.8 else None,
                      bool(rng.random() < 0.5)))
    out = _run(harness, [_plan_line(*c) for c in cases] + ["bad"])
    for c, text in zip(cases, out):
        got = _parse_plan(text)
        want = planner.plan(*c)
        for key in got:
            assert got[key] == want[key], (c, key)
    assert out[-1].startswith("bad 1 invalid argument null output pointer")


def test_cpu_baseline_loops_under_sanitizers(harness):
    rng = np.random.default_rng(4)
    lines, cases = [], []
    for n_dst, n_src, F, threads in ((7, 5, 3, 1), (40, 31, 8, 4), (1, 1, 1, 3), (25, 9, 2, 8)):
        deg = rng.integers(0, 6, size=n_dst)
        rp = np.concatenate([[0], np.cumsum(deg)]).astype(np.int64)
        col = rng.integers(0, n_src, size=int(rp[-1]))
        x = rng.standard_normal((n_src, F)).astype(np.float32)
        w = rng.random(col.size).astype(np.float32)
        dout = rng.standard_normal((n_dst, F)).astype(np.float32)
        nums = [n_dst, n_src, F, threads, *rp, *col, *x.ravel(), *w, *dout.ravel()]
        lines.append("sum " + " ".join(repr(float(v)) if isinstance(v, np.floating) else str(v)
                                       for v in nums))
        cases.append((rp, col, x, w, dout))
    out = _run(harness, lines)
    for (rp, col, x, w, dout), text in zip(cases, out):
        parts = text[len("sum"):].split("|")
        got = [np.array(p.split(), dtype=np.float64) for p in parts]
        e_dx, e_dw = ref.sum_bwd(rp, col, x, w, dout)
        np.testing.assert_allclose(got[0], ref.sum_fwd(rp, col, x, w).ravel(), rtol=1e-5,
                                   atol=1e-6)
        np.testing.assert_allclose(got[1], np.asarray(e_dx).ravel(), rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(got[2], np.asarray(e_dw).ravel(), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("H,D", [(4, 64), (3, 32), (1, 128), (5, 8)])
def test_cpu_twins_under_sanitizers(harness, H, D):
    # Random graphs with split hub rows; 1 and 4 threads must agree bit for
    # bit; broken columns, plans and permutations must be rejected.
    out = _run(harness, [f"twins {11 + H} 1200 {H} {D}"])
    assert out == ["twins ok"], out

"""The span search every kernel uses (knot_spans / knot_span in
torchsplinekan_amd/csrc/kan_spline.h), compiled for the host and checked
against the definition of find_span (csrc/kan_cuda.cu:205-221 of the
reference): the largest m <= nk - 2 with t[m] <= x < t[m+1], the last
non-degenerate span at x == t[nk-1], -1 outside [t[0], t[nk-1]] or for NaN.
Rows with repeated interior and end knots, points on every knot and just
beside it; the four-way interleaved form (the compact input-side product's
epilogue) must give what the single search (basis_grad_compact_kernel)
gives, on unsorted rows too."""

import os
import shutil
import subprocess

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(os.path.dirname(HERE), "torchsplinekan_amd", "csrc")


def _definition(t, x):
    nk = len(t)
    if not (x >= t[0]) or x > t[-1]:
        return -1
    if x == t[-1]:
        m = nk - 2
        while m > 0 and t[m] == t[-1]:
            m -= 1
        return m
    return min(int(np.searchsorted(t, x, side="right")) - 1, nk - 2)


@pytest.fixture(scope="module")
def span_bin(tmp_path_factory):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    out = str(tmp_path_factory.mktemp("span") / "span_check")
    subprocess.run([hipcc, "-x", "hip", "--cuda-host-only", "-O2", "-std=c++17", "-I", CSRC,
                    os.path.join(HERE, "native", "span_check.cpp"), "-o", out], check=True)
    return out


def _rows(nk, rng):
    base = np.sort(rng.uniform(-1, 1, nk)).astype(np.float32).astype(np.float64)
    uni = np.linspace(-1.3, 1.3, nk).astype(np.float32).astype(np.float64)
    if nk < 9:
        return [base, uni]
    rep = base.copy()
    rep[3:6] = rep[3]                 # a repeated interior knot (zero-length spans)
    ends = base.copy()
    ends[:4] = ends[0]                # clamped (repeated) end knots
    ends[-4:] = ends[-1]
    return [base, rep, ends, uni]


def _points(t):
    f32 = lambda v: float(np.float32(v))
    pts = [f32(v) for v in t]
    pts += [float(np.nextafter(np.float32(v), np.float32(-np.inf))) for v in t]
    pts += [float(np.nextafter(np.float32(v), np.float32(np.inf))) for v in t]
    pts += [f32(0.5 * (a + b)) for a, b in zip(t[:-1], t[1:])]
    pts += [f32(t[0] - 1.0), f32(t[-1] + 1.0), float("nan"), float("inf"), float("-inf")]
    return pts


@pytest.mark.parametrize("nk", [2, 3, 9, 17, 33, 72])
def test_span_search_matches_definition(span_bin, nk):
    rng = np.random.default_rng(nk)
    cases = [(t, x) for t in _rows(nk, rng) for x in _points(t)]
    text = f"{nk} {len(cases)}\n" + "\n".join(
        " ".join(repr(float(v)) for v in t) + " " + repr(x) for t, x in cases)
    out = subprocess.run([span_bin], input=text, capture_output=True, text=True, check=True)
    got = np.array([list(map(int, line.split())) for line in out.stdout.split("\n") if line])
    want = np.array([_definition(t, x) for t, x in cases])
    assert got.shape == (len(cases), 4)
    for col in range(4):
        bad = np.nonzero(got[:, col] != want)[0]
        assert bad.size == 0, (col, [(cases[i][1], got[i, col], want[i]) for i in bad[:5]])


def test_interleaved_search_agrees_on_unsorted_rows(span_bin):
    """The epilogue's four-way search and the single search are one routine:
    they return the same span on any row, sorted or not."""
    rng = np.random.default_rng(7)
    nk = 17
    cases = []
    for _ in range(200):
        t = rng.uniform(-1, 1, nk).astype(np.float32).astype(np.float64)
        cases.append((t, float(np.float32(rng.uniform(-1.2, 1.2)))))
    text = f"{nk} {len(cases)}\n" + "\n".join(
        " ".join(repr(float(v)) for v in t) + " " + repr(x) for t, x in cases)
    out = subprocess.run([span_bin], input=text, capture_output=True, text=True, check=True)
    got = np.array([list(map(int, line.split())) for line in out.stdout.split("\n") if line])
    assert np.array_equal(got[:, 2], got[:, 0]) and np.array_equal(got[:, 3], got[:, 0])

"""Re-derives the polynomial of ormi_tanh (ormi_amd/csrc/hip/device/ormi_device.h)
on the host.

For |y| < 0.625 the device computes tanh y = y + y^3 P(y^2), P of degree 4.
P minimises the largest relative error of tanh over [0, 0.625]. With u = y^2
and f(u) = (tanh y - y) / y^3, the relative error is w(u) (P(u) - f(u)) with
w(u) = y^3 / tanh y, a weighted minimax problem in u on [0, 0.390625]. A
discrete Remez exchange on a dense grid solves it here. The test checks that:
  * the solution equioscillates (6 alternating extrema of equal size, one
    more than P has coefficients), the condition that characterises the best
    approximation;
  * its error is the 4.4e-9 the header states;
  * the header's fp32 coefficients are that solution rounded to nearest fp32
    (each within half an fp32 ulp), so their error (8.6e-9, from the rounding
    of the coefficients, 0.14 fp32 ulp) is the rounded solution's.
CPU only; the device rounding of the same formula is tested on the GPU
against float64 (tests/test_hip_parity.py, the tanh ulp sweep)."""
import re
from pathlib import Path

import numpy as np

HEADER = Path(__file__).resolve().parents[1] / "ormi_amd" / "csrc" / "hip" / "device" / "ormi_device.h"
DEG = 4
Y_MAX = 0.625


def header_coefficients():
    """P's coefficients from ormi_tanh's body, constant term first."""
    text = HEADER.read_text()
    body = text[text.index("__device__ __forceinline__ float ormi_tanh(float y)"):]
    body = body[: body.index("}")]
    first = float(re.search(r"float p = (-?[0-9.e+-]+)f;", body).group(1))
    rest = [float(v) for v in re.findall(r"__builtin_fmaf\(p, u, (-?[0-9.e+-]+)f\)", body)]
    hi_to_lo = [first] + rest
    assert len(hi_to_lo) == DEG + 1, hi_to_lo
    return np.array(hi_to_lo[::-1])


def target(u):
    """f(u) = (tanh y - y) / y^3 and the weight y^3 / tanh y, u = y^2; the
    Taylor series of f below y = 0.05 avoids the cancellation of tanh y - y."""
    y = np.sqrt(u)
    small = y < 0.05
    ys = np.where(small, 1.0, y)
    f = np.where(small,
                 -1 / 3 + 2 / 15 * u - 17 / 315 * u ** 2 + 62 / 2835 * u ** 3 - 1382 / 155925 * u ** 4,
                 (np.tanh(ys) - ys) / ys ** 3)
    w = np.where(y > 0, ys ** 3 / np.tanh(ys), 0.0)  # tanh y itself has no cancellation
    w = np.where(small & (y > 0), y ** 3 / np.tanh(np.where(y > 0, y, 1.0)), w)
    return f, w


def rel_error(c, u):
    f, w = target(u)
    return w * (np.polyval(c[::-1], u) - f)


def remez(grid_n=200001, iters=30):
    u = np.linspace(0.0, Y_MAX ** 2, grid_n)
    f, w = target(u)
    n = DEG + 2
    ref = np.linspace(0, grid_n - 1, n).round().astype(int)
    ref[0] = 1  # w(0) = 0: start just inside
    c = np.zeros(DEG + 1)
    for _ in range(iters):
        # P(u_i) + (-1)^i E / w(u_i) = f(u_i) at the reference points
        A = np.zeros((n, n))
        for i, k in enumerate(ref):
            A[i, : DEG + 1] = u[k] ** np.arange(DEG + 1)
            A[i, DEG + 1] = (-1) ** i / w[k]
        sol = np.linalg.solve(A, f[ref])
        c = sol[: DEG + 1]
        err = w * (np.polyval(c[::-1], u) - f)
        # new reference: the extremum of each run of equal sign
        sign = np.sign(err)
        sign[sign == 0] = 1
        edges = np.flatnonzero(np.diff(sign)) + 1
        runs = np.split(np.arange(grid_n), edges)
        peaks = [r[np.argmax(np.abs(err[r]))] for r in runs if len(r)]
        if len(peaks) < n:
            break
        # keep n alternating peaks including the largest
        while len(peaks) > n:
            mags = [abs(err[p]) for p in peaks]
            drop = 0 if mags[0] < mags[-1] else len(peaks) - 1
            peaks.pop(drop)
        ref = np.array(peaks)
    return c, u, w * (np.polyval(c[::-1], u) - f)


def test_remez_solution_equioscillates_at_the_stated_error():
    c, u, err = remez()
    peak = np.max(np.abs(err))
    assert 4.3e-9 < peak < 4.5e-9, peak
    # 7 extrema of alternating sign and (nearly) equal size: the best approximation
    sign = np.sign(err)
    sign[sign == 0] = 1
    runs = np.split(np.arange(len(u)), np.flatnonzero(np.diff(sign)) + 1)
    ext = [np.max(np.abs(err[r])) for r in runs if len(r) > 1]
    assert len(ext) == DEG + 2, len(ext)
    assert min(ext) > 0.98 * peak


def test_header_coefficients_are_the_fit_rounded_to_fp32():
    c_fit, u, err_fit = remez()
    c_hdr = header_coefficients()
    ulp = np.abs(np.spacing(c_fit.astype(np.float32))).astype(np.float64)
    assert np.all(np.abs(c_hdr - c_fit) <= 0.5 * ulp), ((c_hdr - c_fit) / ulp)
    err_round = np.max(np.abs(rel_error(c_fit.astype(np.float32).astype(np.float64), u)))
    err_hdr = np.max(np.abs(rel_error(c_hdr, u)))
    assert err_hdr <= 1.01 * err_round, (err_hdr, err_round)
    assert err_hdr < 2.0 ** -26  # a quarter of an fp32 ulp, relative
    # a plausible slip fails: the two leading coefficients off by 4 fp32 ulps,
    # or the cubic term's Taylor value -1/3 in place of the fitted one
    for k in (0, 1):
        bad = c_hdr.copy()
        bad[k] += 4 * ulp[k]
        assert np.max(np.abs(rel_error(bad, u))) > 1.5 * err_hdr, k
    taylor = c_hdr.copy()
    taylor[0] = -1 / 3
    assert np.max(np.abs(rel_error(taylor, u))) > 10 * err_hdr

"""The Snake forward's sin^2 and the backward's (sin^2, sin 2th) pair, and
the spectral head's (sin, cos) pairs (brosoundml_amd/csrc/kdec_snake_math.hpp),
built for the host with g++ and checked against double precision: the error
bound over wide argument ranges, the values at multiples of pi/2 (every
quadrant's signs), the tiny argument limit and arguments past 2^31. The GPU kernels compile the same header; their forward parity
is in test_gpu_ops.py."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

SRC = r"""
#include <cmath>
#include <cstdio>
#include <random>
#include "kdec_snake_math.hpp"
int main() {
    std::mt19937_64 g(11);
    const double ranges[] = {1.0, 100.0, 30000.0};
    for (double R : ranges) {
        std::uniform_real_distribution<float> U(-R, R);
        double max_abs = 0.0, max_s2 = 0.0, max_sq = 0.0, max_sc = 0.0;
        for (int i = 0; i < 400000; ++i) {
            float th = U(g);
            if (i % 4 == 0)  // next to a multiple of pi/2, where the reduction cancels most
                th = static_cast<float>(std::nearbyint(th / (M_PI / 2)) * (M_PI / 2)) + U(g) * 1e-6f;
            const double ex = std::sin(static_cast<double>(th));
            max_abs = std::fmax(max_abs, std::fabs(kdec::snake_sin2(th) - ex * ex));
            float sq, s2;
            kdec::snake_sin2_sin2x(th, sq, s2);
            max_sq = std::fmax(max_sq, std::fabs(sq - ex * ex));
            max_s2 = std::fmax(max_s2, std::fabs(s2 - std::sin(2.0 * static_cast<double>(th))));
            float sv, cv;
            kdec::kdec_sincos(th, sv, cv);
            max_sc = std::fmax(max_sc, std::fmax(std::fabs(sv - ex), std::fabs(cv - std::cos(static_cast<double>(th)))));
        }
        std::printf("range %g %.6e\n", R, max_abs);
        std::printf("sincos %g %.6e\n", R, max_sc);
        std::printf("pair %g %.6e %.6e\n", R, max_sq, max_s2);
    }
    // past 2^31 the quadrant index exceeds int range: results stay finite and in range
    const float huge[] = {3.0e9f, -7.5e12f, 1.0e30f};
    for (float th : huge) {
        float sq, s2;
        kdec::snake_sin2_sin2x(th, sq, s2);
        std::printf("huge %d\n", std::isfinite(sq) && std::isfinite(s2) && sq >= 0.0f && sq <= 1.0f + 1e-6f &&
                                     std::fabs(s2) <= 1.0f + 1e-6f ? 1 : 0);
    }
    for (int q = -8; q <= 8; ++q) {
        const float th = static_cast<float>(q * (M_PI / 2));
        const double ex = std::sin(static_cast<double>(th));
        std::printf("quad %d %.9e %.9e\n", q, kdec::snake_sin2(th), ex * ex);
        float sv, cv;
        kdec::kdec_sincos(th, sv, cv);
        std::printf("quadsc %d %.9e %.9e %.9e %.9e\n", q, sv, ex, cv, std::cos(static_cast<double>(th)));
    }
    std::printf("tiny %.9e\n", kdec::snake_sin2(1e-10f) / 1e-20);
    {  // the unit-range pair on [-1, 1], its ends, zero and the smallest normal
        std::uniform_real_distribution<float> U(-1.0f, 1.0f);
        double max_u = 0.0;
        for (int i = 0; i < 400000; ++i) {
            float x = U(g);
            if (i == 0) x = 1.0f;
            if (i == 1) x = -1.0f;
            if (i == 2) x = 0.0f;
            if (i == 3) x = 1.17549435e-38f;
            float sv, cv;
            kdec::kdec_sincos_unit(x, sv, cv);
            max_u = std::fmax(max_u, std::fmax(std::fabs(sv - std::sin(static_cast<double>(x))),
                                               std::fabs(cv - std::cos(static_cast<double>(x)))));
        }
        float s0, c0;
        kdec::kdec_sincos_unit(0.0f, s0, c0);
        std::printf("unit %.6e %d\n", max_u, s0 == 0.0f && c0 == 1.0f ? 1 : 0);
    }
    return 0;
}
"""


@pytest.fixture(scope="module")
def results(tmp_path_factory):
    d = tmp_path_factory.mktemp("snake")
    src, exe = d / "t.cpp", d / "t"
    src.write_text(SRC)
    inc = os.path.join(ROOT, "brosoundml_amd", "csrc")
    subprocess.run(["g++", "-O2", "-std=c++17", "-I", inc, str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    return [line.split() for line in out if line]


def test_error_bound(results):
    # the C library's sinf squared reaches ~9e-8 here; the reduced-argument
    # series stays within 2e-7 absolute up to |th| = 30000
    for r in results:
        if r[0] == "range":
            assert float(r[2]) < 2e-7, r


def test_sin2_and_sin2x_pair(results):
    # the backward's pair from one reduction: sin^2 as the forward's, sin 2th
    # (the derivative 1 + sin 2th and the alpha-grad term) within 3e-7
    rows = [r for r in results if r[0] == "pair"]
    assert len(rows) == 3
    for r in rows:
        assert float(r[2]) < 2e-7 and float(r[3]) < 3e-7, r


def test_huge_arguments(results):
    rows = [r for r in results if r[0] == "huge"]
    assert rows and all(r[1] == "1" for r in rows), rows


def test_quadrants(results):
    for r in results:
        if r[0] == "quad":
            got, ref = float(r[2]), float(r[3])
            assert abs(got - ref) < 2e-7, r
            assert (int(r[1]) % 2 == 0) == (got < 0.5), r  # 0 at even multiples, 1 at odd


def test_tiny_argument(results):
    # sin^2(th) / th^2 -> 1
    tiny = [r for r in results if r[0] == "tiny"][0]
    assert abs(float(tiny[1]) - 1.0) < 1e-6


def test_sincos_pair(results):
    # the spectral head's sin and cos from one reduction: within 2e-7 of
    # double up to |th| = 30000, with every quadrant's signs
    rows = [r for r in results if r[0] == "sincos"]
    assert len(rows) == 3
    for r in rows:
        assert float(r[2]) < 2e-7, r
    quads = [r for r in results if r[0] == "quadsc"]
    assert len(quads) == 17
    for r in quads:
        assert abs(float(r[2]) - float(r[3])) < 2e-7 and abs(float(r[4]) - float(r[5])) < 2e-7, r


def test_sincos_unit(results):
    # the spectral head's second map, sin / cos of a sine, by the series
    # without a reduction: within 2e-7 of double over [-1, 1], exact at 0
    row = [r for r in results if r[0] == "unit"][0]
    assert float(row[1]) < 2e-7 and row[2] == "1", row

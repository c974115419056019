"""The Snake forward's sin^2 (brosoundml_amd/csrc/kdec_snake_math.hpp), built
for the host with g++ and checked against double-precision sin^2: the error
bound over wide argument ranges, the values at multiples of pi/2 and the tiny
argument limit. The GPU kernels compile the same header; their forward parity
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
        double max_abs = 0.0;
        for (int i = 0; i < 400000; ++i) {
            float th = U(g);
            if (i % 4 == 0)  // next to a multiple of pi/2, where the reduction cancels most
                th = static_cast<float>(std::nearbyint(th / (M_PI / 2)) * (M_PI / 2)) + U(g) * 1e-6f;
            const double ex = std::sin(static_cast<double>(th));
            max_abs = std::fmax(max_abs, std::fabs(kdec::snake_sin2(th) - ex * ex));
        }
        std::printf("range %g %.6e\n", R, max_abs);
    }
    for (int q = -8; q <= 8; ++q) {
        const float th = static_cast<float>(q * (M_PI / 2));
        const double ex = std::sin(static_cast<double>(th));
        std::printf("quad %d %.9e %.9e\n", q, kdec::snake_sin2(th), ex * ex);
    }
    std::printf("tiny %.9e\n", kdec::snake_sin2(1e-10f) / 1e-20);
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

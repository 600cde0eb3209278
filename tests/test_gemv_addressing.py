"""CPU replay of the GEMV kernel's addressing (cpi_amd/csrc/gemv_plan.hpp,
the same header the kernel includes): no load leaves the weight / scale
buffers and every (row, chunk) is accumulated exactly once, for the shapes
the engine and tests use and for odd shapes, wave shapes and K-splits."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("addr") / "gemv_addr_check")
    subprocess.run(["g++", "-std=c++17", "-O2", "-o", exe, os.path.join(ROOT, "tests", "gemv_addr_check.cpp")],
                   check=True)
    return exe


SHAPES = [(12288, 4096), (22016, 4096), (4096, 11008), (4096, 4096), (32000, 4096), (40, 96), (8, 32),
          (300, 544), (37, 256), (5, 1024), (2048 + 4096 // 8 * 0 + 2560, 2048), (11264, 2048), (2048, 5632),
          (28672, 4096), (4096, 14336), (1, 32), (7, 64), (100, 11008)]


@pytest.mark.parametrize("R,K", SHAPES)
@pytest.mark.parametrize("elems", [8, 16, 32])
def test_addressing_default_plan(checker, R, K, elems):
    if K % elems:
        pytest.skip("K not a multiple of the chunk width")
    out = subprocess.run([checker, str(R), str(K), str(elems), "-1", "0"], capture_output=True, text=True)
    assert out.returncode == 0, out.stdout


@pytest.mark.parametrize("ks", [1, 2, 4])
@pytest.mark.parametrize("shape", range(6))
@pytest.mark.parametrize("R,K", [(300, 544), (4096, 11008), (40, 96), (1000, 4096), (24, 8192)])
def test_addressing_forced(checker, R, K, ks, shape):
    """Every (wave shape, K-split) the kernel can be forced into; invalid
    combinations fall back to a valid plan, which must also be correct."""
    for elems in (8, 16, 32):
        if K % elems:
            continue
        out = subprocess.run([checker, str(R), str(K), str(elems), str(shape), str(ks)], capture_output=True,
                             text=True)
        assert out.returncode == 0, out.stdout

"""Lane layouts of the gfx950 MFMA builtins the DGDA kernels rely on.

Each probe runs one MFMA on per-lane operand registers built from host
matrices under an assumed layout and compares the raw accumulator registers
with the host product (small integers: the fp32 result is exact).
"""
import ctypes
import os

import numpy as np
import pytest
import torch

from conftest import REPO

pytestmark = pytest.mark.gpu
PROBE = os.path.join(REPO, "tests", "hip", "_build", "libmfma_probe.so")


@pytest.fixture(scope="module")
def lib():
    if not (torch.cuda.is_available() and os.path.exists(PROBE)):
        pytest.skip("needs GPU and built probe library")
    lib = ctypes.CDLL(PROBE)
    lib.probe_mfma.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    return lib


def _bf16_bits(x):
    return torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16).view(torch.int16)


def _run(lib, kind, a_regs, b_regs, nout):
    dev = torch.device("cuda:0")
    a = _bf16_bits(a_regs).to(dev)
    b = _bf16_bits(b_regs).to(dev)
    d = torch.zeros(64 * nout, dtype=torch.float32, device=dev)
    rc = lib.probe_mfma(kind, a.data_ptr(), b.data_ptr(), d.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    return d.cpu().numpy().reshape(64, nout)


def test_16x16x16_bf16_layout(lib):
    rng = np.random.default_rng(0)
    A = rng.integers(-4, 5, (16, 16)).astype(np.float32)
    B = rng.integers(-4, 5, (16, 16)).astype(np.float32)
    a_regs = np.zeros((64, 4)); b_regs = np.zeros((64, 4))
    for l in range(64):
        for i in range(4):
            a_regs[l, i] = A[l % 16, 4 * (l // 16) + i]
            b_regs[l, i] = B[4 * (l // 16) + i, l % 16]
    d = _run(lib, 0, a_regs, b_regs, 4)
    C = A @ B
    exp = np.array([[C[4 * (l // 16) + i, l % 16] for i in range(4)] for l in range(64)])
    np.testing.assert_array_equal(d, exp)


def test_16x16x32_bf16_layout(lib):
    rng = np.random.default_rng(1)
    A = rng.integers(-4, 5, (16, 32)).astype(np.float32)
    B = rng.integers(-4, 5, (32, 16)).astype(np.float32)
    a_regs = np.zeros((64, 8)); b_regs = np.zeros((64, 8))
    for l in range(64):
        for i in range(8):
            a_regs[l, i] = A[l % 16, 8 * (l // 16) + i]
            b_regs[l, i] = B[8 * (l // 16) + i, l % 16]
    d = _run(lib, 1, a_regs, b_regs, 4)
    C = A @ B
    exp = np.array([[C[4 * (l // 16) + i, l % 16] for i in range(4)] for l in range(64)])
    np.testing.assert_array_equal(d, exp)


def test_32x32x16_bf16_layout(lib):
    rng = np.random.default_rng(2)
    A = rng.integers(-4, 5, (32, 16)).astype(np.float32)
    B = rng.integers(-4, 5, (16, 32)).astype(np.float32)
    a_regs = np.zeros((64, 8)); b_regs = np.zeros((64, 8))
    for l in range(64):
        for i in range(8):
            a_regs[l, i] = A[l % 32, 8 * (l // 32) + i]
            b_regs[l, i] = B[8 * (l // 32) + i, l % 32]
    d = _run(lib, 2, a_regs, b_regs, 16)
    C = A @ B
    exp = np.array([[C[8 * (i // 4) + 4 * (l // 32) + (i % 4), l % 32] for i in range(16)] for l in range(64)])
    np.testing.assert_array_equal(d, exp)


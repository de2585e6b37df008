"""GPU test of moegemm_matmul_splitk_noalloc through the C ABI (its static scratch area).

Two calls in a row, the second smaller, each compared bit for bit with moegemm_matmul_splitk on a
caller workspace (the same kernels and the same split-order reduction, so the outputs must be
identical), and against a float32 torch product (normwise 1e-2, bf16).  A launch whose partials
do not fit the static area is rejected on the host before anything runs.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from helpers import normwise

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _gpu_only():
    if not torch.cuda.is_available():
        pytest.skip("ROCm GPU unavailable")


# (m, k, n, tile (bm, bn, bk, waves, stages), splits); the second call is smaller than the first.
CALLS = [(64, 4096, 1024, (16, 256, 64, 4, 4), 8), (16, 2048, 512, (16, 256, 64, 4, 4), 4)]


def _args(a, b, c, tile, splits):
    from kernels import _native

    bm, bn, bk, warps, stages = tile
    m, k = a.shape
    n = b.shape[1]
    return (a.data_ptr(), b.data_ptr(), c.data_ptr(), m, n, k, a.stride(0), a.stride(1), b.stride(0), b.stride(1),
            c.stride(0), c.stride(1), _native.DTYPE_BF16, bm, bn, bk, 8, warps, stages, splits, 0)


def test_noalloc_splitk_matches_the_workspace_entry_point_twice():
    from kernels import _native

    lib = _native.library()
    stream = _native.current_stream_handle(torch.device("cuda"))
    generator = torch.Generator(device="cuda").manual_seed(17)
    for m, k, n, tile, splits in CALLS:
        print(f"noalloc split-K m={m} k={k} n={n} tile={tile} splits={splits}", flush=True)
        a = torch.randn((m, k), device="cuda", generator=generator).div_(k ** 0.5).to(torch.bfloat16)
        b = torch.randn((k, n), device="cuda", generator=generator).to(torch.bfloat16)
        expected = torch.full((m, n), float("nan"), device="cuda", dtype=torch.bfloat16)
        got = torch.full((m, n), float("nan"), device="cuda", dtype=torch.bfloat16)
        tiles = -(-m // tile[0]) * -(-n // tile[1])
        nbytes = _native.splitk_workspace_bytes(tiles, splits, tile[0], tile[1])
        workspace = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
        _native.check(lib.moegemm_matmul_splitk(*_args(a, b, expected, tile, splits), workspace.data_ptr(),
                                                workspace.numel(), 0, stream))
        _native.check(lib.moegemm_matmul_splitk_noalloc(*_args(a, b, got, tile, splits), 0, stream))
        torch.cuda.synchronize()
        assert torch.isfinite(got).all()
        assert torch.equal(got, expected)
        assert normwise(got, a.float() @ b.float()) <= 1e-2


def test_noalloc_splitk_rejects_partials_beyond_the_static_area():
    from kernels import _native

    lib = _native.library()
    a = torch.zeros((4096, 4096), device="cuda", dtype=torch.bfloat16)
    b = torch.zeros((4096, 4096), device="cuda", dtype=torch.bfloat16)
    c = torch.zeros((4096, 4096), device="cuda", dtype=torch.bfloat16)
    status = lib.moegemm_matmul_splitk_noalloc(*_args(a, b, c, (256, 256, 64, 8, 2), 4),
                                               0, ctypes.c_void_p(_native.current_stream_handle(a.device)))
    assert status == _native.ERR_INVALID
    assert "static area" in _native.last_error()
    torch.cuda.synchronize()
    assert not c.any()  # nothing ran

"""GPU parity tests: the HIP kernels (through the C ABI) against the CPU oracle.

Mirrors the reference's tests/test_gpu.py cases (odd shapes in three dtypes, strided fp32/TF32,
heterogeneous distinct pointers, homogeneous fast path, exact-integer known answers for every
candidate, multi-round persistent grid with NaN guard bands, packed W13, G == 1 dispatch) and
adds the BASELINE.json shapes.  Tolerances: exact integers are compared bit for bit; random inputs
use the reference's per-dtype ``assert_close`` and the normwise bound max|C - R| / max|R|
(bf16 <= 1e-2, fp16 <= 2e-3, fp32 <= 1e-5) against the oracle's fp64-accumulated product.
"""

from __future__ import annotations

import math

import pytest
import torch

from helpers import DTYPE_NAME, normwise, oracle_product

pytestmark = pytest.mark.gpu

NORMWISE = {"bf16": 1e-2, "fp16": 2e-3, "fp32": 1e-5}
DTYPES = (torch.float16, torch.bfloat16, torch.float32)


@pytest.fixture(autouse=True)
def _gpu_only():
    if not torch.cuda.is_available():
        pytest.skip("ROCm GPU unavailable")
    torch.manual_seed(7)
    from utils.benchmark import configure_torch_matmul

    configure_torch_matmul("ieee")


def _check(actual: torch.Tensor, a: torch.Tensor, b: torch.Tensor, *, tf32: bool = False) -> None:
    from utils.benchmark import assert_close

    name = DTYPE_NAME[a.dtype]
    expected = oracle_product(a, b, tf32=tf32)
    assert torch.isfinite(actual).all()
    assert normwise(actual, expected) <= NORMWISE[name]
    assert_close(actual.cpu(), expected.to(actual.dtype), name)


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: DTYPE_NAME[d])
def test_single_odd_shapes_all_dtypes(dtype):
    from kernels.matmul import last_matmul_config, launch_matmul, select_config

    for m, k, n in ((1, 5, 3), (17, 13, 31), (33, 70, 65)):
        print(f"single odd shape m={m} k={k} n={n} dtype={DTYPE_NAME[dtype]}", flush=True)
        a = torch.randn((m, k), device="cuda", dtype=dtype) * 0.1
        b = torch.randn((k, n), device="cuda", dtype=dtype) * 0.1
        c = torch.full((m, n), float("nan"), device="cuda", dtype=dtype)
        fallback = select_config(m, n, k, dtype)
        launch_matmul(a, b, c, fallback)
        torch.cuda.synchronize()
        selected = last_matmul_config(fallback)
        assert selected.block_m in (16, 32, 64, 128, 256)
        assert selected.block_n in (32, 64, 128, 256)
        assert selected.block_k in (32, 64, 128)
        _check(c, a, b)


def test_single_strided_fp32_tf32():
    from kernels.matmul import launch_matmul

    m, k, n = 17, 70, 65
    a = (torch.randn((m, k * 2), device="cuda") * 0.1)[:, ::2]
    b = (torch.randn((k, n * 2), device="cuda") * 0.1)[:, ::2]
    storage = torch.full((m, n * 2), float("nan"), device="cuda")
    c = storage[:, ::2]
    launch_matmul(a, b, c, input_precision="tf32")
    torch.cuda.synchronize()
    _check(c, a, b, tf32=True)
    assert torch.isnan(storage[:, 1::2]).all(), "strided store touched the gaps between columns"


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: DTYPE_NAME[d])
def test_grouped_distinct_pointers_shapes_and_dtypes(dtype):
    from kernels.grouped_gemm import build_grouped_workspace, launch_grouped
    from kernels.matmul import select_config

    shapes = [(1, 5, 3), (17, 13, 31), (9, 70, 65)]
    workspace = build_grouped_workspace(shapes, dtype, seed=99, config=select_config(17, 65, 70, dtype))
    assert len({x.data_ptr() for x in workspace.a}) == len(shapes)
    launch_grouped(workspace)
    torch.cuda.synchronize()
    assert workspace.scheduler == "generic_persistent"
    for a, b, c in workspace.problem_tensors():
        _check(c, a, b)


def test_grouped_homogeneous_persistent_fast_path():
    from kernels.grouped_gemm import build_grouped_workspace, launch_grouped

    workspace = build_grouped_workspace([(17, 13, 31)] * 3, torch.float16, seed=101)
    assert workspace.homogeneous
    launch_grouped(workspace)
    torch.cuda.synchronize()
    assert workspace.scheduler == "homogeneous_persistent"
    for a, b, c in workspace.problem_tensors():
        _check(c, a, b)


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: DTYPE_NAME[d])
@pytest.mark.parametrize("shape", [(1, 1, 1), (17, 33, 65), (40, 256, 320)])
def test_homogeneous_every_candidate_exact_integers(dtype, shape):
    """A = 1, B_e = e + 1  =>  C_e == k * (e + 1) exactly, for every candidate config."""
    from kernels.grouped_gemm import build_grouped_workspace, grouped_candidate_configs, launch_grouped

    workspace = build_grouped_workspace([shape] * 3, dtype)
    for index, (a, b, _) in enumerate(workspace.problem_tensors()):
        a.fill_(1)
        b.fill_(index + 1)
    m, k, n = shape
    candidates = grouped_candidate_configs(m, n, k, problem_count=3, sm_count=workspace.sm_count, dtype=dtype)
    assert candidates
    for config in candidates:
        print(f"exact-integer shape={shape} dtype={DTYPE_NAME[dtype]} config={config}", flush=True)
        for output in workspace.c:
            output.fill_(float("nan"))
        launch_grouped(workspace, config=config, autotune=False)
        torch.cuda.synchronize()
        for index, output in enumerate(workspace.c):
            torch.testing.assert_close(output, torch.full_like(output, k * (index + 1)), rtol=0, atol=0)


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: DTYPE_NAME[d])
def test_every_compiled_tile_exact_integers_generic(dtype):
    """Every compiled tile of the dtype, generic mode with ragged shapes: exact integer results."""
    from kernels.grouped_gemm import build_grouped_workspace, launch_grouped
    from kernels.matmul import config_pool

    shapes = [(5, 40, 24), (70, 96, 136), (33, 64, 72), (130, 200, 264)]
    workspace = build_grouped_workspace(shapes, dtype, seed=3)
    assert not workspace.homogeneous
    for index, (a, b, _) in enumerate(workspace.problem_tensors()):
        a.copy_(torch.randint(-2, 3, a.shape, device="cuda").to(dtype))
        b.copy_(torch.randint(-2, 3, b.shape, device="cuda").to(dtype))
    # Integer sums are exact in the fp32 accumulator; the store rounds them to the dtype.
    expected = [(a.double() @ b.double()).to(dtype).double() for a, b, _ in workspace.problem_tensors()]
    tiles = {cfg.tile_key: cfg for cfg in config_pool(dtype) if cfg.group_size_m == 4}
    for cfg in tiles.values():
        print(f"generic exact dtype={DTYPE_NAME[dtype]} config={cfg}", flush=True)
        for output in workspace.c:
            output.fill_(float("nan"))
        launch_grouped(workspace, config=cfg, autotune=False)
        torch.cuda.synchronize()
        for output, ref in zip(workspace.c, expected):
            torch.testing.assert_close(output.double(), ref, rtol=0, atol=0)


def test_homogeneous_persistent_multiple_rounds_and_guard_storage():
    from kernels.grouped_gemm import build_grouped_workspace, launch_grouped
    from kernels.matmul import KernelConfig

    config = KernelConfig(16, 64, 32, 4, 4, 2)
    sm_count = torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count
    m, k, n = (sm_count + 1) * config.block_m + 1, 33, 65
    workspace = build_grouped_workspace([(m, k, n)] * 2, torch.float32)
    guards = []
    for index in range(workspace.problem_count):
        storage = torch.full((m * n + 32,), float("nan"), device=workspace.c[index].device)
        output = storage[16:-16].view(m, n)
        guards.append(storage)
        workspace.c[index] = output
        workspace.c_ptrs[index] = output.data_ptr()
    launch_grouped(workspace, config=config, autotune=False)
    torch.cuda.synchronize()
    for (a, b, c), storage in zip(workspace.problem_tensors(), guards):
        reference = (a.double() @ b.double()).float()
        torch.testing.assert_close(c, reference, rtol=1e-4, atol=1e-6)
        assert torch.isnan(storage[:16]).all()
        assert torch.isnan(storage[-16:]).all()


def test_fused_gate_up_packed_output_in_one_grouped_launch():
    from kernels.grouped_gemm import build_fused_gate_up_workspace, launch_grouped

    local_ffn = 31
    workspace = build_fused_gate_up_workspace([(17, 13, 2 * local_ffn)] * 3, torch.float16, seed=102)
    assert workspace.operation == "gate_up"
    launch_grouped(workspace)
    torch.cuda.synchronize()
    assert workspace.scheduler == "homogeneous_persistent"
    for a, packed_weight, packed_output in workspace.problem_tensors():
        gate = oracle_product(a, packed_weight[:, :local_ffn])
        up = oracle_product(a, packed_weight[:, local_ffn:])
        reference = torch.cat((gate, up), dim=1)
        assert normwise(packed_output, reference) <= NORMWISE["fp16"]


def test_one_problem_group_dispatches_standard_matmul():
    from kernels.grouped_gemm import build_grouped_workspace, launch_grouped

    workspace = build_grouped_workspace([(17, 70, 65)], torch.float16, seed=103)
    launch_grouped(workspace)
    torch.cuda.synchronize()
    assert workspace.scheduler == "single_problem_matmul"
    _check(workspace.c[0], workspace.a[0], workspace.b[0])


def test_plumbing_case_bf16_against_oracle():
    """8 experts of [64, 512] @ [512, 1024], bf16, N(0,1)/sqrt(K) inputs."""
    from kernels.grouped_gemm import launch_grouped, workspace_from_tensors

    g, m, k, n = 8, 64, 512, 1024
    gen = torch.Generator(device="cpu").manual_seed(1234)
    a = [(torch.randn((m, k), generator=gen) / math.sqrt(k)).to(torch.bfloat16).cuda() for _ in range(g)]
    b = [(torch.randn((k, n), generator=gen) / math.sqrt(k)).to(torch.bfloat16).cuda() for _ in range(g)]
    c = [torch.full((m, n), float("nan"), device="cuda", dtype=torch.bfloat16) for _ in range(g)]
    workspace = workspace_from_tensors(a, b, c)
    launch_grouped(workspace)
    torch.cuda.synchronize()
    assert workspace.scheduler == "homogeneous_persistent"
    for ai, bi, ci in workspace.problem_tensors():
        _check(ci, ai, bi)

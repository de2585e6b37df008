"""Expert-sorted grouped GEMM (2-D A, 3-D B, int32 offsets) on gfx950.

The layout a router produces after token permutation: one expert-sorted A [rows, K], the expert
weights as one B [G, K, N], and int32 cumulative end rows ``offs`` [G], so that group e owns rows
offs[e-1]:offs[e] of A and C.  This is the operand layout of the reference's torch provider
(kernels/torch_grouped_gemm.py:121-174: ``build_torch_grouped_workspace`` pads row strides to 16 B
and calls ``torch.nn.functional.grouped_mm(mat_a, mat_b, offs=offs)`` once).  Here the same
operands go to the persistent HIP kernel through ``moegemm_grouped_mm_offs``:

* ``grouped_mm(mat_a, mat_b, offs, out=None)`` has the 2-D x 3-D semantics of
  ``torch.nn.functional.grouped_mm`` (C[offs[e-1]:offs[e]] = A[offs[e-1]:offs[e]] @ B[e], fp32
  accumulation, output in the operand dtype).  ``offs`` stays on the device: the kernel derives
  every group's row count from it at run time, so the call needs no host synchronisation and is
  capturable in a HIP graph (one kernel launch).  Rows at or past offs[-1] are not written (torch
  leaves them unspecified too: ``out=None`` allocates with ``torch.empty`` like torch); offsets
  beyond ``rows`` are clamped on the device, so any ``offs`` content is memory-safe (offsets that
  decrease give empty or overlapping groups, whose results are unspecified).
* ``grouped_mm_swiglu`` is the packed Gate+Up launch over the same layout with the SiLU(gate)*up
  activation fused into the epilogue (H [rows, F] out; one kernel launch).
* ``build_offsets_workspace`` / ``launch_grouped_offsets`` mirror the torch provider's workspace
  API for the drivers (same seeded ``normal_() * 0.1`` operands, same 16-byte row padding, same
  ``problem_tensors()`` view of each expert).
"""

from __future__ import annotations

from collections.abc import Iterator, Sequence
from dataclasses import dataclass
from itertools import accumulate

from . import _native
from .grouped_gemm import grouped_candidate_configs
from .matmul import KernelConfig, _device_signature, _require_runtime, _tune, config_pool, select_config


def offsets_tile_bound(rows: int, group_count: int, n: int, block_m: int, block_n: int) -> int:
    """Host-side upper bound of the tile count the kernel may find in ``offs`` (mirrors the C ABI).

    Each group contributes at most one partial M tile, and no group has more rows than A.
    """
    if rows <= 0:
        return 0
    m_tiles = min(rows // block_m + group_count, group_count * -(-rows // block_m))
    return m_tiles * -(-n // block_n)


def _validate(mat_a, mat_b, offs, out):
    import torch

    if mat_a.ndim != 2 or mat_b.ndim != 3:
        raise ValueError("grouped_mm expects a 2-D mat_a [rows, K] and a 3-D mat_b [G, K, N]")
    rows, k = mat_a.shape
    groups, kb, n = mat_b.shape
    if k != kb:
        raise ValueError(f"contraction mismatch: mat_a K={k}, mat_b K={kb}")
    if offs.ndim != 1 or offs.dtype != torch.int32 or offs.shape[0] != groups:
        raise ValueError(f"offs must be an int32 vector with one entry per group ({groups})")
    if not offs.is_contiguous():
        # The kernel reads offs[e] as a dense int32 array from its base address: a strided view
        # would give wrong group boundaries and an expanded one would read past its storage.
        raise ValueError("offs must be contiguous (pass offs.contiguous())")
    if groups <= 0 or k <= 0 or n <= 0:
        raise ValueError("grouped_mm needs at least one group and positive K and N")
    devices = {mat_a.device, mat_b.device, offs.device}
    if out is not None:
        devices.add(out.device)
    if len(devices) != 1 or mat_a.device.type != "cuda":
        raise ValueError("mat_a, mat_b, offs and out must be on the same GPU device")
    if mat_a.dtype != mat_b.dtype:
        raise ValueError("mat_a and mat_b must have the same dtype")
    if mat_a.stride(1) != 1 or mat_b.stride(2) != 1:
        raise ValueError("mat_a and mat_b need a unit stride along their last dimension")
    if out is not None:
        if tuple(out.shape) != (rows, n) or out.dtype != mat_a.dtype or out.stride(1) != 1:
            raise ValueError(f"out must be a [{rows}, {n}] {mat_a.dtype} matrix with unit column stride")
    return int(rows), int(k), int(n), int(groups)


def _launch_fixed(mat_a, mat_b, offs, out, rows, k, n, groups, cfg: KernelConfig, dtype_code: int,
                  precision: int, sm_count: int, schedule: str = "static", b_stream: int = 0) -> None:
    grid = max(1, min(offsets_tile_bound(rows, groups, n, cfg.block_m, cfg.block_n), sm_count * cfg.cta_multiplier))
    stream = _native.current_stream_handle(mat_a.device)
    args = (
        mat_a.data_ptr(), mat_b.data_ptr(), out.data_ptr(), offs.data_ptr(), groups, rows, n, k,
        mat_a.stride(0), mat_b.stride(0), mat_b.stride(1), out.stride(0), dtype_code, precision,
        cfg.block_m, cfg.block_n, cfg.block_k, cfg.group_size_m, cfg.num_warps, cfg.num_stages, grid,
    )
    if schedule == "stealing":
        queue = _native.tile_queue(mat_a.device, stream)
        status = _native.library().moegemm_grouped_mm_offs_stealing(*args, queue.data_ptr(), b_stream, stream)
    else:
        status = _native.library().moegemm_grouped_mm_offs(*args, b_stream, stream)
    _native.check(status)


_OFFSETS_AUTOTUNE_CACHE: dict[tuple, tuple[KernelConfig, str, int]] = {}
_LAST_CONFIG: list[KernelConfig | None] = [None]
_LAST_SCHEDULE: list[str] = ["static"]
_LAST_B_STREAM: list[int] = [0]


def last_grouped_mm_config() -> KernelConfig | None:
    """Config used by the most recent ``grouped_mm`` call."""
    return _LAST_CONFIG[0]


def last_grouped_mm_schedule() -> str:
    """Tile schedule ("static" or "stealing") of the most recent ``grouped_mm`` call."""
    return _LAST_SCHEDULE[0]


def last_grouped_mm_b_stream() -> int:
    """B copy policy of the most recent ``grouped_mm`` call: 1 = non-temporal B copies."""
    return _LAST_B_STREAM[0]


def grouped_mm(mat_a, mat_b, offs, *, out=None, config: KernelConfig | None = None,
               input_precision: str = "ieee", autotune: bool = True, tile_schedule: str | None = None,
               b_stream: int | None = None):
    """C = per-group A @ B[e] over the expert-sorted layout; returns ``out`` (allocated if None).

    With ``autotune=True`` and no ``config``, the first call per (rows, K, N, G, strides, dtype)
    key measures the candidate tiles on these operands; later calls are a cache lookup plus one
    kernel launch.  The tuning key does not include ``offs``: the candidates are ranked for an
    even split of ``rows`` over the groups.  ``tile_schedule``: "static", "stealing" (per-XCD
    work-stealing tile queues), or None to let the tuner measure both (static otherwise).
    ``b_stream``: 1 issues the LDS-DMA kernels' B copies non-temporal, 0 as ordinary loads, None lets
    the tuner measure both on its finalists (0 without autotuning).
    """
    import torch

    if tile_schedule is not None and tile_schedule not in _native.TILE_SCHEDULES:
        raise ValueError(f"tile_schedule must be None or one of {_native.TILE_SCHEDULES}, got {tile_schedule!r}")
    if b_stream not in (None, 0, 1):
        raise ValueError(f"b_stream must be None, 0 or 1, got {b_stream!r}")
    rows, k, n, groups = _validate(mat_a, mat_b, offs, out)
    _require_runtime()
    if out is None:
        out = torch.empty((rows, n), device=mat_a.device, dtype=mat_a.dtype)
    if rows == 0:
        return out
    dtype_code = _native.dtype_code(mat_a.dtype)
    precision = _native.precision_code(input_precision, dtype_code)
    sm_count = _device_signature(mat_a.device) % 1000
    mean_m = max(1, rows // groups)

    def launch(option):
        _launch_fixed(mat_a, mat_b, offs, out, rows, k, n, groups, option[0], dtype_code, precision, sm_count,
                      option[1], option[2])

    if config is not None or not autotune:
        option = (config or select_config(mean_m, n, k, mat_a.dtype), tile_schedule or "static", b_stream or 0)
    else:
        key = (rows, k, n, groups, tuple(mat_a.stride()), tuple(mat_b.stride()), tuple(out.stride()),
               dtype_code, precision, _device_signature(mat_a.device), tile_schedule, b_stream)
        option = _OFFSETS_AUTOTUNE_CACHE.get(key)
        if option is None:
            candidates = grouped_candidate_configs(mean_m, n, k, problem_count=max(groups, 2), sm_count=sm_count,
                                                   dtype=mat_a.dtype)
            schedules = _native.TILE_SCHEDULES if tile_schedule is None else (tile_schedule,)
            options = [(cfg, schedule, b_stream or 0) for cfg in candidates for schedule in schedules]
            # The B copy policy is timed on the finalists where it is not pinned (16-bit operands; the
            # general kernel ignores it).
            sixteen = mat_a.dtype in (torch.float16, torch.bfloat16)
            twin = (lambda o: (o[0], o[1], 1)) if b_stream is None and sixteen else None
            option = _tune(options, launch, twin=twin)
            _OFFSETS_AUTOTUNE_CACHE[key] = option
    launch(option)
    _LAST_CONFIG[0], _LAST_SCHEDULE[0], _LAST_B_STREAM[0] = option
    return out


_SWIGLU_OFFSETS_CACHE: dict[tuple, KernelConfig] = {}
_LAST_SWIGLU_CONFIG: list[KernelConfig | None] = [None]


def last_grouped_mm_swiglu_config() -> KernelConfig | None:
    """Config used by the most recent ``grouped_mm_swiglu`` call."""
    return _LAST_SWIGLU_CONFIG[0]


def grouped_mm_swiglu(mat_a, mat_b, offs, *, out=None, config: KernelConfig | None = None,
                      autotune: bool = True):
    """Packed Gate+Up with the SwiGLU activation fused, over the expert-sorted layout.

    ``mat_b`` [G, K, 2F] holds each group's [gate | up] columns (the packed W13 weights of the
    reference's build_fused_gate_up_workspace, kernels/grouped_gemm.py:575-594, in the 3-D layout
    of its torch provider).  Returns H [rows, F] with H[r0:r1] = silu(A[r0:r1] @ B[e][:, :F]) *
    (A[r0:r1] @ B[e][:, F:]) computed from the fp32 accumulators, for r0 = offs[e-1] (0 for e = 0)
    and r1 = offs[e].  One kernel launch; rows at or past offs[-1] are not written.  fp16/bf16 in
    the vector layout (16-byte aligned rows, K and F multiples of 8) only (ValueError otherwise).
    Autotuning as in ``grouped_mm``, over the tiles that can pair gate and up fragments.
    """
    import torch

    rows, k, n, groups = _validate(mat_a, mat_b, offs, None)
    f = n // 2
    if mat_a.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("the fused SwiGLU epilogue needs fp16 or bf16 operands")
    if n % 16:
        raise ValueError(f"packed Gate+Up width must be 2F with F a multiple of 8 (got {n} columns)")
    if out is not None and (tuple(out.shape) != (rows, f) or out.dtype != mat_a.dtype or out.stride(1) != 1
                            or out.device != mat_a.device):
        raise ValueError(f"out must be a [{rows}, {f}] {mat_a.dtype} matrix with unit column stride on the same device")
    vector = (k % 8 == 0 and mat_a.stride(0) % 8 == 0 and mat_b.stride(1) % 8 == 0 and mat_b.stride(0) % 8 == 0
              and mat_a.data_ptr() % 16 == 0 and mat_b.data_ptr() % 16 == 0)
    if not vector:
        raise ValueError("the fused SwiGLU epilogue needs 16-byte aligned operands with K a multiple of 8")
    _require_runtime()
    if out is None:
        out = torch.empty((rows, f), device=mat_a.device, dtype=mat_a.dtype)
    if out.stride(0) % 4 or out.data_ptr() % 8:
        raise ValueError("out rows must be 8-byte aligned")
    if rows == 0:
        return out
    dtype_code = _native.dtype_code(mat_a.dtype)
    sm_count = _device_signature(mat_a.device) % 1000
    allowed = _native.swiglu_tiles(dtype_code)

    def launch(cfg):
        grid = max(1, min(offsets_tile_bound(rows, groups, n, cfg.block_m, cfg.block_n), sm_count * cfg.cta_multiplier))
        status = _native.library().moegemm_grouped_mm_offs_swiglu(
            mat_a.data_ptr(), mat_b.data_ptr(), out.data_ptr(), offs.data_ptr(), groups, rows, n, k,
            mat_a.stride(0), mat_b.stride(0), mat_b.stride(1), out.stride(0), dtype_code,
            cfg.block_m, cfg.block_n, cfg.block_k, cfg.group_size_m, cfg.num_warps, cfg.num_stages, grid,
            0, _native.current_stream_handle(mat_a.device),
        )
        _native.check(status)

    if config is not None or not autotune:
        cfg = config
        if cfg is None:
            cfg = next((c for c in config_pool(mat_a.dtype) if c.tile_key in allowed and c.group_size_m == 8), None)
    else:
        key = (rows, k, n, groups, tuple(mat_a.stride()), tuple(mat_b.stride()), tuple(out.stride()), dtype_code,
               _device_signature(mat_a.device))
        cfg = _SWIGLU_OFFSETS_CACHE.get(key)
        if cfg is None:
            mean_m = max(1, rows // groups)
            ranked = grouped_candidate_configs(mean_m, n, k, problem_count=max(groups, 2), sm_count=sm_count,
                                               dtype=mat_a.dtype)
            candidates = [c for c in ranked if c.tile_key in allowed] or \
                [c for c in config_pool(mat_a.dtype) if c.tile_key in allowed and c.group_size_m == 8][:6]
            cfg = _tune(candidates, launch)
            _SWIGLU_OFFSETS_CACHE[key] = cfg
    launch(cfg)
    _LAST_SWIGLU_CONFIG[0] = cfg
    return out


@dataclass
class OffsetsWorkspace:
    mat_a: object
    mat_b: object
    offs: object
    shapes: tuple[tuple[int, int, int], ...]
    output: object
    config: KernelConfig
    sm_count: int = 0
    device_signature: int = 0
    operation: str = "gemm"
    scheduler: str = "not_launched"
    tile_schedule: str = "static"

    @property
    def problem_count(self) -> int:
        return len(self.shapes)

    @property
    def storage_bytes(self) -> int:
        tensors = (self.mat_a, self.mat_b, self.offs, self.output)
        return sum(t.untyped_storage().nbytes() for t in tensors)

    def problem_tensors(self) -> Iterator[tuple[object, object, object]]:
        row = 0
        for index, (m, _, _) in enumerate(self.shapes):
            yield self.mat_a[row:row + m], self.mat_b[index], self.output[row:row + m]
            row += m


def build_offsets_workspace(
    shapes: Sequence[tuple[int, int, int]],
    dtype,
    seed: int = 0,
    *,
    operation: str = "gemm",
    device: str = "cuda",
) -> OffsetsWorkspace:
    """Expert-sorted operands for (M_e, K, N) problems sharing K and N (16-byte padded rows)."""
    import torch

    if not shapes:
        raise ValueError("grouped GEMM requires at least one problem")
    normalized = tuple(tuple(int(v) for v in s) for s in shapes)
    if any(len(s) != 3 or s[0] < 0 or s[1] <= 0 or s[2] <= 0 for s in normalized):
        raise ValueError("every shape must be an (M >= 0, K > 0, N > 0) triple")
    _, k, n = normalized[0]
    if any(kk != k or nn != n for _, kk, nn in normalized):
        raise ValueError("the expert-sorted layout requires shared K and N dimensions")
    ends = tuple(accumulate(m for m, _, _ in normalized))
    if ends[-1] > 2**31 - 1:
        raise ValueError("offsets exceed int32 range")
    per16 = max(1, 16 // torch.empty((), dtype=dtype).element_size())

    def padded(extent: int) -> int:
        return -(-extent // per16) * per16

    generator = torch.Generator(device=device).manual_seed(seed)
    rows = ends[-1]
    mat_a = torch.empty((rows, padded(k)), device=device, dtype=dtype)[:, :k]
    mat_b = torch.empty((len(normalized), k, padded(n)), device=device, dtype=dtype)[:, :, :n]
    mat_a.normal_(generator=generator).mul_(0.1)
    mat_b.normal_(generator=generator).mul_(0.1)
    output = torch.empty((rows, padded(n)), device=device, dtype=dtype)[:, :n]
    offs = torch.tensor(ends, device=device, dtype=torch.int32)
    config = select_config(max(1, rows // len(normalized)), n, k, dtype)
    signature = _device_signature(mat_a.device) if mat_a.device.type == "cuda" else 0
    return OffsetsWorkspace(mat_a, mat_b, offs, normalized, output, config, sm_count=signature % 1000,
                            device_signature=signature, operation=operation)


def launch_grouped_offsets(workspace: OffsetsWorkspace, input_precision: str = "ieee",
                           config: KernelConfig | None = None, *, autotune: bool = True,
                           tile_schedule: str | None = None) -> None:
    """One persistent kernel over the workspace; records the config, scheduler name and tile schedule.

    Like ``launch_grouped``: with ``autotune=True`` the per-workload tuner picks the config (an
    explicit ``config`` is ignored); otherwise ``config`` (or the workspace's) runs as given.
    """
    grouped_mm(workspace.mat_a, workspace.mat_b, workspace.offs, out=workspace.output,
               config=None if autotune else (config or workspace.config),
               input_precision=input_precision, autotune=autotune, tile_schedule=tile_schedule)
    workspace.config = last_grouped_mm_config()
    workspace.scheduler = "offsets_persistent"
    workspace.tile_schedule = last_grouped_mm_schedule()

"""CPU tests that pin the oracle before it is trusted as the GPU checker.

Each oracle function is checked against something it did not produce:
  * golden vectors from torch CPU float64 (tests/golden/gemm_golden.npz, make_golden.py);
  * closed forms (A = 1, B = e + 1 => C = k (e + 1), the reference's known-answer test,
    tests/test_gpu.py:127-154) and a pure-Python brute force on tiny shapes;
  * numpy float64 matmul for strided views, torch / numpy casts for the rounding functions;
  * planted mistakes (a transposed operand, a dropped K term, a shifted column, dims in (m, k, n)
    order, swapped strides, pointer tables out of step): each must fail the same comparison that
    the oracle passes, so the comparison has teeth.
A last test checks that every public oracle function and every symbol of liboracle.so is called
here.
"""

from __future__ import annotations

import itertools
import math
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle

GOLDEN = np.load(Path(__file__).resolve().parent / "golden" / "gemm_golden.npz", allow_pickle=False)


def _values(bits_or_f32: np.ndarray, dtype: str) -> np.ndarray:
    return oracle.to_float(np.asarray(bits_or_f32), dtype).astype(np.float64)


@pytest.mark.parametrize("name", [str(n) for n in GOLDEN["case_names"]])
def test_gemm_matches_torch_float64_golden(name):
    dtype = name.split("_")[0]
    a, b = GOLDEN[f"{name}_a"], GOLDEN[f"{name}_b"]
    out, sums = oracle.gemm(a, b, dtype, return_sums=True)
    exact = GOLDEN[f"{name}_exact"]
    if dtype == "fp32":
        np.testing.assert_allclose(sums, exact, rtol=1e-12, atol=1e-15)
        np.testing.assert_allclose(out, exact.astype(np.float32), rtol=2e-7, atol=1e-12)
    else:
        # Products of 16-bit values are exact and these sums fit a double: bit-exact both ways.
        np.testing.assert_array_equal(sums, exact)
        np.testing.assert_array_equal(out, GOLDEN[f"{name}_out"])


def test_w13_packed_matches_golden_and_split_form():
    a, b = GOLDEN["w13_fp16_a"], GOLDEN["w13_fp16_b"]
    packed = oracle.gemm(a, b, "fp16")
    np.testing.assert_array_equal(packed, GOLDEN["w13_fp16_out"])
    np.testing.assert_array_equal(oracle.w13_reference(a, b, "fp16"), packed)


def test_plumbing_case_sample_matches_golden():
    a, bcols = GOLDEN["plumbing_a"], GOLDEN["plumbing_b_cols"]
    rows = GOLDEN["plumbing_rows"]
    out, sums = oracle.gemm(a, bcols, "bf16", return_sums=True)
    picked = sums[rows, np.arange(len(rows))]
    np.testing.assert_array_equal(picked, GOLDEN["plumbing_exact"])
    np.testing.assert_array_equal(out[rows, np.arange(len(rows))], GOLDEN["plumbing_out"])


@pytest.mark.parametrize("dtype", ["fp16", "bf16", "fp32"])
@pytest.mark.parametrize("shape", [(1, 1, 1), (17, 33, 65), (3, 200, 7)])
def test_known_answer_ones_times_index(dtype, shape):
    m, k, n = shape
    store = np.float32 if dtype == "fp32" else np.uint16
    one = np.ones(1, np.float32)
    encode = {"bf16": oracle.to_bf16_bits, "fp16": oracle.to_f16_bits, "fp32": lambda v: v.astype(np.float32)}[dtype]
    a = np.full((m, k), encode(one)[0], dtype=store)
    for e in range(3):
        b = np.full((k, n), encode(np.array([e + 1.0], np.float32))[0], dtype=store)
        out = oracle.gemm(a, b, dtype)
        expected = np.full((m, n), k * (e + 1), dtype=np.float64)
        np.testing.assert_array_equal(_values(out, dtype), _values(encode(expected.astype(np.float32)), dtype))


def _brute(a_vals, b_vals):
    m, k = len(a_vals), len(a_vals[0])
    n = len(b_vals[0])
    return [[math.fsum(a_vals[i][l] * b_vals[l][j] for l in range(k)) for j in range(n)] for i in range(m)]


@pytest.mark.parametrize("dtype", ["fp16", "bf16", "fp32"])
def test_brute_force_tiny(dtype):
    rng = np.random.default_rng(5)
    for m, k, n in [(1, 1, 1), (2, 3, 4), (5, 7, 3)]:
        av = rng.standard_normal((m, k)).astype(np.float32)
        bv = rng.standard_normal((k, n)).astype(np.float32)
        if dtype == "fp32":
            a, b = av, bv
        else:
            enc = oracle.to_bf16_bits if dtype == "bf16" else oracle.to_f16_bits
            a, b = enc(av), enc(bv)
        _, sums = oracle.gemm(a, b, dtype, return_sums=True)
        expect = _brute(_values(a, dtype).tolist(), _values(b, dtype).tolist())
        np.testing.assert_allclose(sums, np.array(expect), rtol=1e-13, atol=1e-13)


def test_strided_views_match_numpy():
    rng = np.random.default_rng(9)
    base_a = rng.standard_normal((17, 140)).astype(np.float32)
    base_b = rng.standard_normal((70, 130)).astype(np.float32)
    a, b = base_a[:, ::2], base_b[:, ::2]  # non-unit inner strides
    _, sums = oracle.gemm(a, b, "fp32", return_sums=True)
    np.testing.assert_allclose(sums, a.astype(np.float64) @ b.astype(np.float64), rtol=1e-12, atol=1e-12)
    bt = np.ascontiguousarray(base_b[:, :65].T).T  # column-major B
    _, sums_t = oracle.gemm(a, bt, "fp32", return_sums=True)
    np.testing.assert_allclose(sums_t, a.astype(np.float64) @ bt.astype(np.float64), rtol=1e-12, atol=1e-12)


def test_fp32_accumulation_model_differs_only_by_rounding():
    name = "bf16_40x256x320"
    a, b = GOLDEN[f"{name}_a"], GOLDEN[f"{name}_b"]
    _, s64 = oracle.gemm(a, b, "bf16", return_sums=True)
    _, s32 = oracle.gemm(a, b, "bf16", accum="f32", return_sums=True)
    scale = np.abs(s64).max()
    assert 0 < np.abs(s32 - s64).max() / scale < 256 * 2.0**-24


# ---------------------------------------------------------------------------------------------
# Planted mistakes: the comparisons above must reject plausible implementation errors.

def _mutant_transposed(a, b, dtype):
    n = min(b.shape)
    sq = np.ascontiguousarray(b[:n, :n].T)
    return oracle.gemm(np.ascontiguousarray(a[:, :n]), sq, dtype)


@pytest.mark.parametrize("mutant", ["transposed_b", "dropped_k_term", "shifted_column"])
def test_planted_mistakes_fail_the_golden_comparison(mutant):
    name = "fp16_33x70x65"
    a, b = GOLDEN[f"{name}_a"], GOLDEN[f"{name}_b"]
    good = GOLDEN[f"{name}_out"]
    if mutant == "transposed_b":
        got = _mutant_transposed(a, b, "fp16")
        assert got.shape != good.shape or not np.array_equal(got, good)
        sq_a, sq_b = a[:, :65], b[:65, :65]
        np.testing.assert_raises(AssertionError, np.testing.assert_array_equal,
                                 oracle.gemm(np.ascontiguousarray(sq_a), np.ascontiguousarray(sq_b.T), "fp16"),
                                 oracle.gemm(np.ascontiguousarray(sq_a), np.ascontiguousarray(sq_b), "fp16"))
    elif mutant == "dropped_k_term":
        got = oracle.gemm(np.ascontiguousarray(a[:, :-1]), np.ascontiguousarray(b[:-1]), "fp16")
        assert not np.array_equal(got, good)
    else:
        got = oracle.gemm(a, b, "fp16")
        assert not np.array_equal(np.roll(got, 1, axis=1), good)


# ---------------------------------------------------------------------------------------------
# Rounding

def test_bf16_rounding_matches_torch_casts():
    values = GOLDEN["round_values"]
    np.testing.assert_array_equal(oracle.to_bf16_bits(values), GOLDEN["round_bf16"])


def test_fp16_rounding_matches_torch_and_numpy_casts():
    values = GOLDEN["round_values"]
    got = oracle.to_f16_bits(values)
    np.testing.assert_array_equal(got, GOLDEN["round_fp16"])
    with np.errstate(over="ignore"):  # values past the half range must become +-inf
        np.testing.assert_array_equal(got, values.astype(np.float16).view(np.uint16))


def test_bf16_nan_stays_nan_and_decoders_are_exact():
    nan_bits = oracle.to_bf16_bits(np.array([np.nan], np.float32))
    assert np.isnan(oracle.bf16_bits_to_float(nan_bits))[0]
    all_f16 = np.arange(0, 65536, dtype=np.uint32).astype(np.uint16)
    finite = (all_f16 & 0x7C00) != 0x7C00
    np.testing.assert_array_equal(oracle.f16_bits_to_float(all_f16)[finite],
                                  all_f16.view(np.float16).astype(np.float32)[finite])


def test_tf32_rounding_ties_away_and_truncation_grid():
    ulp = 2.0**-10
    cases = {
        1.0: 1.0,
        1.0 + ulp / 2: 1.0 + ulp,          # tie -> away from zero
        -(1.0 + ulp / 2): -(1.0 + ulp),
        1.0 + ulp / 2 - 2.0**-23: 1.0,     # just below the tie -> down
        1.0 + 3 * ulp / 2: 1.0 + 2 * ulp,  # tie -> away (not to even)
    }
    got = oracle.tf32_round(np.array(list(cases), np.float32))
    np.testing.assert_array_equal(got, np.array(list(cases.values()), np.float32))
    rng = np.random.default_rng(3)
    x = rng.standard_normal(1000).astype(np.float32)
    assert np.all((oracle.tf32_round(x).view(np.uint32) & 0x1FFF) == 0)


# ---------------------------------------------------------------------------------------------
# Tables and launch rules (kernels/grouped_gemm.py:530-552, 597-640)

def test_tables_order_and_dispatch_rules():
    shapes = [(1, 5, 3), (17, 13, 31), (9, 70, 65)]
    dims, strides = oracle.tables(shapes)
    assert dims.tolist() == [[1, 3, 5], [17, 31, 13], [9, 65, 70]]
    assert strides.tolist()[1] == [13, 1, 31, 1, 31, 1]
    assert oracle.dispatch(1, True) == "single_problem_matmul"
    assert oracle.dispatch(3, True) == "homogeneous_persistent"
    assert oracle.dispatch(3, False) == "generic_persistent"
    assert oracle.is_homogeneous([(17, 13, 31)] * 3, [True] * 9)
    assert not oracle.is_homogeneous(shapes, [True] * 9)
    assert not oracle.is_homogeneous([(17, 13, 31)] * 3, [True] * 8 + [False])
    # (1,5,3): 1x1 tiles; (17,13,31): 2x1; (9,70,65): 1x2.
    assert oracle.grid_size(shapes, 16, 64, 120, 2) == 1 + 2 + 2
    assert oracle.grid_size([(4096, 8, 4096)] * 4, 128, 128, 120, 2) == 240


@pytest.mark.parametrize("m_tiles,n_tiles,group_m", [(1, 1, 8), (5, 3, 2), (9, 4, 4), (16, 7, 8), (3, 5, 1)])
def test_group_m_tile_walks_bands_column_major(m_tiles, n_tiles, group_m):
    # The traversal as nested loops: bands of group_m M tiles (the last one shorter); inside a
    # band, N tiles in order and, for each, the band's M tiles in order.
    expected = []
    for first in range(0, m_tiles, group_m):
        band = range(first, min(first + group_m, m_tiles))
        expected += [(tm, tn) for tn in range(n_tiles) for tm in band]
    got = [oracle.group_m_tile(t, m_tiles, n_tiles, group_m) for t in range(m_tiles * n_tiles)]
    assert got == expected
    if group_m > 1 and m_tiles > 1 and n_tiles > 1:  # a planted row-major band order differs
        row_major = [(tm, tn) for first in range(0, m_tiles, group_m)
                     for tm in range(first, min(first + group_m, m_tiles)) for tn in range(n_tiles)]
        assert got != row_major


@pytest.mark.parametrize("group_m", [1, 4, 8])
@pytest.mark.parametrize("grid", [1, 7, 64])
def test_tile_order_visits_every_tile_once(group_m, grid):
    shapes = [(1, 5, 3), (130, 40, 300), (64, 8, 64), (257, 9, 129)]
    visits = oracle.tile_order(shapes, 64, 64, group_m, grid)
    flat = list(itertools.chain.from_iterable(visits))
    expected = {(e, tm, tn) for e, (m, _, n) in enumerate(shapes)
                for tm in range(math.ceil(m / 64)) for tn in range(math.ceil(n / 64))}
    assert len(flat) == len(expected) == oracle.tile_count(shapes, 64, 64)
    assert set(flat) == expected


# --------------------------------------------------------------------------------------------
# Grouped table form: pointer tables, dims (m, n, k), strides (am, ak, bk, bn, cm, cn)
# (reference kernels/grouped_gemm.py:427-449 reads them, :530-544 builds them)

@pytest.mark.parametrize("dtype", ["fp16", "bf16", "fp32"])
def test_grouped_gemm_heterogeneous_group_matches_golden(dtype):
    names = [n for n in map(str, GOLDEN["case_names"]) if n.startswith(dtype + "_")]
    assert len(names) >= 3
    a_list = [GOLDEN[f"{n}_a"] for n in names]
    b_list = [GOLDEN[f"{n}_b"] for n in names]
    outs = oracle.grouped_gemm(a_list, b_list, dtype)
    for name, out in zip(names, outs):
        if dtype == "fp32":
            np.testing.assert_allclose(out, GOLDEN[f"{name}_exact"].astype(np.float32), rtol=2e-7, atol=1e-12)
        else:
            np.testing.assert_array_equal(out, GOLDEN[f"{name}_out"])
    # The grouped form agrees bit for bit with the single-problem form in both accumulation models.
    for accum in ("f64", "f32"):
        single = [oracle.gemm(a, b, dtype, accum=accum) for a, b in zip(a_list, b_list)]
        for got, want in zip(oracle.grouped_gemm(a_list, b_list, dtype, accum=accum), single):
            np.testing.assert_array_equal(got, want)


_PAD = 4096  # every operand lives inside a zero-padded buffer, so planted table mistakes stay in bounds


def _strided_group(dtype):
    """Three heterogeneous problems, each with a different stride pattern, as (buffers, tables,
    expected C).  Operand values are small integers, so every sum is exact before its one rounding."""
    rng = np.random.default_rng(31)
    store = np.float32 if dtype == "fp32" else np.uint16
    encode = {"bf16": oracle.to_bf16_bits, "fp16": oracle.to_f16_bits,
              "fp32": lambda v: np.asarray(v, np.float32)}[dtype]
    problems = [(5, 7, 3), (17, 13, 31), (9, 20, 6)]  # (m, k, n): n != k everywhere
    a_bufs, b_bufs, c_bufs, dims, strides, expect = [], [], [], [], [], []
    for p, (m, k, n) in enumerate(problems):
        av = rng.integers(-4, 5, (m, k)).astype(np.float32)
        bv = rng.integers(-4, 5, (k, n)).astype(np.float32)
        abuf = np.zeros(_PAD, store)
        bbuf = np.zeros(_PAD, store)
        if p == 0:    # A with a non-unit inner stride, B column-major, C column-major
            am, ak, bk, bn, cm, cn = 2 * k, 2, 1, k, 1, m
        elif p == 1:  # contiguous A, B rows padded past n, C rows padded past n
            am, ak, bk, bn, cm, cn = k, 1, n + 9, 1, n + 5, 1
        else:         # A transposed (column-major), B with both strides non-unit, C row-major
            am, ak, bk, bn, cm, cn = 1, m, 2 * n + 1, 2, n, 1
        for i in range(m):
            for l in range(k):
                abuf[i * am + l * ak] = encode(np.array([av[i, l]], np.float32))[0]
        for l in range(k):
            for j in range(n):
                bbuf[l * bk + j * bn] = encode(np.array([bv[l, j]], np.float32))[0]
        a_bufs.append(abuf)
        b_bufs.append(bbuf)
        c_bufs.append(np.zeros(_PAD, store))
        dims.append((m, n, k))
        strides.append((am, ak, bk, bn, cm, cn))
        exact = np.array(_brute(av.tolist(), bv.tolist()), dtype=np.float32)
        expect.append(_values(encode(exact), dtype))  # one rounding, by the casts pinned above
    return a_bufs, b_bufs, c_bufs, dims, strides, expect


def _gather_c(cbuf, dims_e, strides_e, dtype):
    m, n, _ = dims_e
    cm, cn = strides_e[4], strides_e[5]
    idx = np.arange(m)[:, None] * cm + np.arange(n)[None, :] * cn
    return _values(cbuf[idx], dtype)


@pytest.mark.parametrize("dtype", ["fp16", "bf16", "fp32"])
def test_grouped_gemm_tables_strided_heterogeneous_matches_brute_force(dtype):
    a_bufs, b_bufs, c_bufs, dims, strides, expect = _strided_group(dtype)
    oracle.grouped_gemm_tables(a_bufs, b_bufs, c_bufs, dims, strides, dtype)
    for e in range(3):
        np.testing.assert_array_equal(_gather_c(c_bufs[e], dims[e], strides[e], dtype), expect[e])
        # Nothing outside the strided C footprint is written.
        m, n, _ = dims[e]
        cm, cn = strides[e][4], strides[e][5]
        mask = np.ones(_PAD, bool)
        mask[(np.arange(m)[:, None] * cm + np.arange(n)[None, :] * cn).ravel()] = False
        assert not np.any(c_bufs[e][mask])


@pytest.mark.parametrize("mistake", ["dims_m_k_n", "dims_n_m_k", "strides_ak_am", "strides_bn_bk",
                                     "b_table_rotated"])
def test_grouped_gemm_tables_planted_mistakes_fail(mistake):
    dtype = "bf16"
    a_bufs, b_bufs, c_bufs, dims, strides, expect = _strided_group(dtype)
    dims_bad = [list(d) for d in dims]
    strides_bad = [list(s) for s in strides]
    b_bad = list(b_bufs)
    if mistake == "dims_m_k_n":        # the reference's shape order (m, k, n) instead of (m, n, k)
        dims_bad = [[m, k, n] for m, n, k in dims]
    elif mistake == "dims_n_m_k":
        dims_bad = [[n, m, k] for m, n, k in dims]
    elif mistake == "strides_ak_am":   # A's two strides swapped
        strides_bad = [[s[1], s[0], *s[2:]] for s in strides]
    elif mistake == "strides_bn_bk":   # B's two strides swapped
        strides_bad = [[s[0], s[1], s[3], s[2], s[4], s[5]] for s in strides]
    else:                              # pointer tables out of step with each other
        b_bad = b_bufs[1:] + b_bufs[:1]
    oracle.grouped_gemm_tables(a_bufs, b_bad, c_bufs, dims_bad, strides_bad, dtype)
    mismatched = 0
    for e in range(3):
        got = _gather_c(c_bufs[e], dims[e], strides[e], dtype)
        mismatched += not np.array_equal(got, expect[e])
    assert mismatched >= 1


def test_grouped_gemm_tables_reject_bad_tables():
    a_bufs, b_bufs, c_bufs, dims, strides, _ = _strided_group("fp16")
    with pytest.raises(ValueError):
        oracle.grouped_gemm_tables(a_bufs, b_bufs, c_bufs, [d[:2] for d in dims], strides, "fp16")
    with pytest.raises(ValueError):
        oracle.grouped_gemm_tables([], [], [], np.zeros((0, 3)), np.zeros((0, 6)), "fp16")
    with pytest.raises(ValueError):
        oracle.grouped_gemm(a_bufs[:1], [], "fp16")


def test_c_decoders_exhaustive():
    every = np.arange(0, 65536, dtype=np.uint32).astype(np.uint16)
    got16 = oracle.c_decode(every, "fp16")
    want16 = every.view(np.float16).astype(np.float32)
    finite = np.isfinite(want16)
    np.testing.assert_array_equal(got16[finite], want16[finite])
    assert np.array_equal(np.isnan(got16), np.isnan(want16)) and np.array_equal(np.isinf(got16), np.isinf(want16))
    gotb = oracle.c_decode(every, "bf16")
    wantb = (every.astype(np.uint32) << 16).view(np.float32)
    np.testing.assert_array_equal(gotb.view(np.uint32)[~np.isnan(wantb)], wantb.view(np.uint32)[~np.isnan(wantb)])
    assert np.array_equal(np.isnan(gotb), np.isnan(wantb))


def test_every_oracle_function_and_export_is_exercised_here():
    """Every public function of oracle.py, and every symbol liboracle.so exports, is called by a
    test in this file (so no part of the checker goes unpinned)."""
    import inspect
    import re
    import subprocess

    source = Path(__file__).read_text()
    called = set(re.findall(r"oracle\.(\w+)\(", source))
    public = {name for name, obj in vars(oracle).items()
              if inspect.isfunction(obj) and obj.__module__ == oracle.__name__ and not name.startswith("_")}
    helpers = {"lib"}  # the loader; every test goes through it
    assert public - called - helpers == set()
    exported = subprocess.run(["nm", "-D", "--defined-only", str(oracle.LIBRARY)], check=True,
                              capture_output=True, text=True).stdout
    symbols = {line.split()[-1] for line in exported.splitlines() if " T " in line}
    bound = set(re.findall(r"handle\.(oracle_\w+)\.argtypes", Path(oracle.__file__).read_text()))
    assert symbols and symbols == bound
    # Each bound symbol is reached through a function this file calls.
    reaches = {"oracle_gemm": "gemm", "oracle_grouped_gemm": "grouped_gemm_tables",
               "oracle_gemm_rowmajor_fast": "gemm_fast_bf16", "oracle_float_to_bf16": "to_bf16_bits",
               "oracle_float_to_f16": "to_f16_bits", "oracle_tf32_round": "tf32_round",
               "oracle_f16_to_float": "c_decode", "oracle_bf16_to_float": "c_decode"}
    assert set(reaches) == symbols
    assert set(reaches.values()) <= called


# --------------------------------------------------------------------------------------------
# Expert-sorted layout (2-D A, 3-D B, int32 offsets)

def _torch_cpu_grouped_mm(a_bits, b_bits, offs, dtype):
    import torch

    tdt = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}[dtype]
    if dtype == "fp32":
        ta, tb = torch.from_numpy(np.ascontiguousarray(a_bits)), torch.from_numpy(np.ascontiguousarray(b_bits))
    else:
        ta = torch.from_numpy(np.ascontiguousarray(a_bits).view(np.int16)).view(tdt)
        tb = torch.from_numpy(np.ascontiguousarray(b_bits).view(np.int16)).view(tdt)
    out = torch.nn.functional.grouped_mm(ta, tb, offs=torch.tensor(offs, dtype=torch.int32))
    return out.float().numpy().astype(np.float64)


@pytest.mark.parametrize("dtype", ["bf16", "fp16", "fp32"])
def test_grouped_mm_offsets_matches_torch_cpu_grouped_mm(dtype):
    rng = np.random.default_rng(7)
    rows, k, n = 37, 48, 24
    offs = [5, 5, 19, 30]  # an empty group and rows 30..36 past the last offset
    af = rng.standard_normal((rows, k)).astype(np.float32) / math.sqrt(k)
    bf = rng.standard_normal((len(offs), k, n)).astype(np.float32) / math.sqrt(k)
    enc = {"bf16": oracle.to_bf16_bits, "fp16": oracle.to_f16_bits, "fp32": lambda x: x}[dtype]
    a, b = enc(af), enc(bf)
    ours = _values(oracle.grouped_mm_offsets(a, b, offs, dtype), dtype)
    theirs = _torch_cpu_grouped_mm(a, b, offs, dtype)
    # torch accumulates in float32, the oracle in float64: 16-bit outputs are at most one output
    # rounding step apart; fp32 outputs differ by float32 accumulation error (k terms, normwise).
    ulp = {"bf16": 2.0 ** -7, "fp16": 2.0 ** -10, "fp32": 2.0 ** -21}[dtype]
    scale = float(np.abs(theirs[:30]).max())
    atol = k * 2.0 ** -24 * scale if dtype == "fp32" else ulp * 1e-2
    # Rows past offs[-1] are unspecified in torch (left uninitialised); the oracle leaves zeros.
    np.testing.assert_allclose(ours[:30], theirs[:30], rtol=ulp, atol=atol)
    assert np.all(ours[30:] == 0)


def test_grouped_mm_offsets_brute_force_and_planted_shift():
    rng = np.random.default_rng(3)
    rows, k, n = 9, 5, 3
    offs = [2, 6, 9]
    a = rng.standard_normal((rows, k)).astype(np.float32)
    b = rng.standard_normal((3, k, n)).astype(np.float32)
    got = oracle.grouped_mm_offsets(a, b, offs, "fp32").astype(np.float64)
    brute = np.zeros((rows, n))
    starts = [0] + offs[:-1]
    for e, (lo, hi) in enumerate(zip(starts, offs)):
        for r in range(lo, hi):
            for j in range(n):
                brute[r, j] = math.fsum(float(a[r, t]) * float(b[e, t, j]) for t in range(k))
    np.testing.assert_allclose(got, brute, rtol=1e-6, atol=1e-6)
    shifted = oracle.grouped_mm_offsets(a, b, [3, 6, 9], "fp32").astype(np.float64)  # planted: one row moved
    assert not np.allclose(shifted, brute, rtol=1e-6, atol=1e-6)


def test_offsets_groups_clamps_into_the_matrix():
    assert oracle.offsets_groups([3, 3, 7], 10) == [(0, 3), (3, 0), (3, 4)]
    assert oracle.offsets_groups([4, 2, 15], 10) == [(0, 4), (4, 0), (2, 8)]
    assert oracle.offsets_groups([-5, 20], 10) == [(0, 0), (0, 10)]
    for offs in ([3, 3, 7], [4, 2, 15], [-5, 20], [12, 12]):
        for lo, m in oracle.offsets_groups(offs, 10):
            assert 0 <= lo and lo + m <= 10


@pytest.mark.parametrize("block_m,block_n", [(16, 64), (64, 128), (256, 256)])
def test_offsets_tile_bound_covers_every_split(block_m, block_n):
    n = 300
    for rows in range(0, 43, 7):
        for groups in (1, 2, 3, 4):
            bound = oracle.offsets_tile_bound(rows, groups, n, block_m, block_n)
            # every monotone split of rows into `groups` pieces (exhaustive over cut points)
            for cuts in itertools.combinations_with_replacement(range(rows + 1), groups - 1):
                ends = list(cuts) + [rows]
                tiles = sum(math.ceil(m / block_m) for _, m in oracle.offsets_groups(ends, rows)) * math.ceil(n / block_n)
                assert tiles <= bound


# --------------------------------------------------------------------------------------------
# Fused SwiGLU epilogue over packed Gate+Up weights

@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_swiglu_reference_matches_torch_float64(dtype):
    import torch

    rng = np.random.default_rng(21)
    m, k, f = 13, 40, 24
    enc = {"bf16": oracle.to_bf16_bits, "fp16": oracle.to_f16_bits}[dtype]
    a = enc(rng.standard_normal((m, k)).astype(np.float32))
    b = enc(rng.standard_normal((k, 2 * f)).astype(np.float32) * 0.5)
    ours = _values(oracle.swiglu_reference(a, b, dtype), dtype)
    ta = torch.from_numpy(_values(a, dtype))
    tb = torch.from_numpy(_values(b, dtype))
    theirs = (torch.nn.functional.silu(ta @ tb[:, :f]) * (ta @ tb[:, f:])).numpy()
    ulp = {"bf16": 2.0 ** -8, "fp16": 2.0 ** -11}[dtype]  # half an output ulp: one correct rounding
    np.testing.assert_allclose(ours, theirs, rtol=ulp, atol=1e-30)
    swapped = _values(oracle.swiglu_reference(a, np.concatenate([b[:, f:], b[:, :f]], axis=1), dtype), dtype)
    assert not np.allclose(swapped, theirs, rtol=1e-2, atol=1e-3)  # planted: gate and up exchanged
    with pytest.raises(ValueError):
        oracle.swiglu_reference(a, b[:, :-1], dtype)


# ---------------------------------------------------------------------------------------------
# The OpenMP fp32-accumulating GEMM (``gemm_fast_bf16``), used only to time a CPU baseline.

def _sequential_f32_reference(a_bits: np.ndarray, b_bits: np.ndarray, dtype: str) -> np.ndarray:
    """numpy float32 running sum over k in index order (each 16-bit product is exact in float32),
    rounded to the 16-bit dtype by torch's cast: an implementation independent of the C oracle."""
    import torch

    a = _values(a_bits, dtype).astype(np.float32)
    b = _values(b_bits, dtype).astype(np.float32)
    acc = np.zeros((a.shape[0], b.shape[1]), dtype=np.float32)
    for index in range(a.shape[1]):
        acc = acc + a[:, index:index + 1] * b[index:index + 1, :]
    torch_dtype = torch.bfloat16 if dtype == "bf16" else torch.float16
    return torch.from_numpy(acc).to(torch_dtype).view(torch.int16).numpy().view(np.uint16)


_FAST_SHAPES = [(1, 5, 3), (17, 13, 31), (33, 70, 65), (19, 200, 300), (40, 256, 320), (3, 1000, 257)]


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
@pytest.mark.parametrize("shape", _FAST_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_fast_gemm_is_bit_equal_to_sequential_f32_sums(dtype, shape):
    """Ragged m and n (not multiples of the 16 x 256 blocks) and K not a multiple of 16."""
    m, k, n = shape
    rng = np.random.default_rng(m * 1000 + k + n)
    to_bits = oracle.to_bf16_bits if dtype == "bf16" else oracle.to_f16_bits
    a = to_bits(rng.standard_normal((m, k)).astype(np.float32) / math.sqrt(k))
    b = to_bits(rng.standard_normal((k, n)).astype(np.float32))
    fast = oracle.gemm_fast_bf16(a, b, 4, dtype)
    np.testing.assert_array_equal(fast, _sequential_f32_reference(a, b, dtype))
    np.testing.assert_array_equal(fast, oracle.gemm(a, b, dtype, accum="f32"))


@pytest.mark.parametrize("name", [n for n in map(str, GOLDEN["case_names"]) if not n.startswith("fp32")])
def test_fast_gemm_within_f32_accumulation_bound_of_golden(name):
    """Against the torch float64 golden sums: the difference is at most the float32 running-sum
    error k * 2^-24 * sum|a||b| plus one output rounding of the 16-bit dtype."""
    dtype = name.split("_")[0]
    a, b = GOLDEN[f"{name}_a"], GOLDEN[f"{name}_b"]
    exact = GOLDEN[f"{name}_exact"]
    fast = _values(oracle.gemm_fast_bf16(a, b, 2, dtype), dtype)
    k = a.shape[1]
    magnitude = np.abs(_values(a, dtype)) @ np.abs(_values(b, dtype))
    unit = 2.0**-8 if dtype == "bf16" else 2.0**-11
    bound = k * 2.0**-24 * magnitude + unit * np.abs(exact) + 1e-30
    assert np.all(np.abs(fast - exact) <= bound)
    # Rounded outputs agree with the golden ones except where the f32 sum crosses a rounding edge.
    assert np.mean(oracle.gemm_fast_bf16(a, b, 2, dtype) == GOLDEN[f"{name}_out"]) > 0.9


def test_fast_gemm_planted_dropped_term_fails():
    m, k, n = 16, 64, 128
    rng = np.random.default_rng(5)
    a = oracle.to_bf16_bits(rng.standard_normal((m, k)).astype(np.float32))
    b = oracle.to_bf16_bits(rng.standard_normal((k, n)).astype(np.float32))
    fast = oracle.gemm_fast_bf16(a, b, 2)
    dropped = oracle.gemm_fast_bf16(np.ascontiguousarray(a[:, 1:]), np.ascontiguousarray(b[1:]), 2)
    assert not np.array_equal(fast, dropped)
    assert not np.array_equal(dropped, _sequential_f32_reference(a, b, "bf16"))

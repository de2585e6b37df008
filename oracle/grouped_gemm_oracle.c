/*
 * CPU ORACLE - TEST INFRASTRUCTURE ONLY.
 *
 * Plain-C restatement of the arithmetic of the reference's grouped / single GEMM path, used by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker.  The product
 * path (libmoegemm) never links, loads or calls this code.
 *
 * Reference semantics restated here:
 *   - kernels/grouped_gemm.py:399-482 (_generic_grouped_kernel_impl): for each problem e with
 *     dims[e] = (m, n, k) (order built at :536) and strides[e] = (am, ak, bk, bn, cm, cn)
 *     (order built at :537-544), C_e[i, j] = sum_l A_e[i, l] * B_e[l, j];
 *   - kernels/grouped_gemm.py:321-397 (homogeneous) is the same sum with contiguous strides;
 *   - kernels/matmul.py:223-273 (_matmul_kernel_impl): fp32 accumulator (:256), result cast to
 *     C's dtype on store (:269-273), masked tails contribute nothing (:258-267);
 *   - input_precision "tf32" (the tl.dot argument, kernels/matmul.py:268) rounds fp32 operands to
 *     a 10-bit mantissa.
 * Products of two fp16/bf16 values are exact in fp32; the sum is accumulated in double
 * (accum = ORACLE_ACCUM_F64, the tight reference) or sequentially in float
 * (ORACLE_ACCUM_F32, the reference's fp32-accumulated model), then rounded to nearest-even.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define ORACLE_F16 0
#define ORACLE_BF16 1
#define ORACLE_F32 2
#define ORACLE_ACCUM_F64 0
#define ORACLE_ACCUM_F32 1

static float bits_to_float(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static uint32_t float_to_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

/* IEEE binary16 -> float (exact). */
float oracle_f16_to_float(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  int exp = (h >> 10) & 0x1f;
  uint32_t mant = h & 0x3ffu;
  if (exp == 0x1f) return bits_to_float(sign | 0x7f800000u | (mant << 13));
  double mag = exp == 0 ? ldexp((double)mant, -24) : ldexp(1024.0 + mant, exp - 25);
  float f = (float)mag; /* exact: at most 11 significant bits */
  return sign ? -f : f;
}

/* bfloat16 -> float (exact: the high half of a binary32). */
float oracle_bf16_to_float(uint16_t b) { return bits_to_float((uint32_t)b << 16); }

/* float -> bfloat16, round to nearest even; NaN stays NaN. */
uint16_t oracle_float_to_bf16(float f) {
  uint32_t u = float_to_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* float -> IEEE binary16, round to nearest even, overflow to infinity, gradual underflow. */
uint16_t oracle_float_to_f16(float f) {
  uint32_t u = float_to_bits(f);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  if ((u & 0x7f800000u) == 0x7f800000u) return sign | 0x7c00u | ((u & 0x7fffffu) ? 0x0200u : 0u);
  double x = fabs((double)f);
  if (x >= 65520.0) return sign | 0x7c00u; /* rounds past the largest finite half (65504) */
  if (x < ldexp(1.0, -14)) {               /* subnormal half: multiples of 2^-24 */
    double q = rint(ldexp(x, 24));          /* ties to even under the default rounding mode */
    return sign | (uint16_t)q;              /* q == 1024 is the smallest normal, as it should be */
  }
  int e2;
  double m = frexp(x, &e2); /* x = m * 2^e2, m in [0.5, 1) */
  double q = rint(ldexp(m, 11)) - 1024.0; /* 10 fraction bits of the [1, 2) significand */
  int biased = e2 - 1 + 15;
  if (q >= 1024.0) {
    q = 0.0;
    biased += 1;
  }
  if (biased >= 31) return sign | 0x7c00u;
  return sign | (uint16_t)((biased << 10) | (int)q);
}

/* TF32 operand rounding: nearest, ties away from zero, to a 10-bit mantissa. */
float oracle_tf32_round(float f) {
  uint32_t u = float_to_bits(f);
  if ((u & 0x7f800000u) == 0x7f800000u) return f;
  return bits_to_float((u + 0x1000u) & 0xffffe000u);
}

static float load_elem(const void* base, int64_t index, int dtype, int tf32) {
  if (dtype == ORACLE_F16) return oracle_f16_to_float(((const uint16_t*)base)[index]);
  if (dtype == ORACLE_BF16) return oracle_bf16_to_float(((const uint16_t*)base)[index]);
  float f = ((const float*)base)[index];
  return tf32 ? oracle_tf32_round(f) : f;
}

static void store_elem(void* base, int64_t index, int dtype, double v) {
  if (dtype == ORACLE_F16)
    ((uint16_t*)base)[index] = oracle_float_to_f16((float)v);
  else if (dtype == ORACLE_BF16)
    ((uint16_t*)base)[index] = oracle_float_to_bf16((float)v);
  else
    ((float*)base)[index] = (float)v;
}

/*
 * One problem: C[i*cm + j*cn] = round(sum_l A[i*am + l*ak] * B[l*bk + j*bn]).
 * If acc_out is non-null, the unrounded sums are also written there (row-major m x n doubles).
 */
int oracle_gemm(const void* a, const void* b, void* c, int32_t m, int32_t n, int32_t k, int64_t am, int64_t ak,
                int64_t bk, int64_t bn, int64_t cm, int64_t cn, int32_t dtype, int32_t tf32, int32_t accum,
                double* acc_out) {
  if (m < 0 || n < 0 || k < 0 || dtype < 0 || dtype > 2) return -1;
  for (int32_t i = 0; i < m; ++i) {
    for (int32_t j = 0; j < n; ++j) {
      double s64 = 0.0;
      float s32 = 0.0f;
      for (int32_t l = 0; l < k; ++l) {
        float x = load_elem(a, (int64_t)i * am + (int64_t)l * ak, dtype, tf32);
        float y = load_elem(b, (int64_t)l * bk + (int64_t)j * bn, dtype, tf32);
        if (accum == ORACLE_ACCUM_F32)
          s32 = s32 + x * y;
        else
          s64 += (double)x * (double)y;
      }
      double v = accum == ORACLE_ACCUM_F32 ? (double)s32 : s64;
      if (acc_out) acc_out[(int64_t)i * n + j] = v;
      /* The accumulator is fp32 on the device: round the exact sum to float before the cast. */
      store_elem(c, (int64_t)i * cm + (int64_t)j * cn, dtype, (double)(float)v);
    }
  }
  return 0;
}

/* Grouped form over host pointer tables and the reference's dims/strides tables. */
int oracle_grouped_gemm(int32_t problem_count, const void* const* a_ptrs, const void* const* b_ptrs,
                        void* const* c_ptrs, const int32_t* dims, const int64_t* strides, int32_t dtype,
                        int32_t tf32, int32_t accum) {
  if (problem_count <= 0) return -1;
  for (int32_t e = 0; e < problem_count; ++e) {
    const int32_t* d = dims + 3 * (int64_t)e;
    const int64_t* s = strides + 6 * (int64_t)e;
    int rc = oracle_gemm(a_ptrs[e], b_ptrs[e], c_ptrs[e], d[0], d[1], d[2], s[0], s[1], s[2], s[3], s[4], s[5], dtype,
                         tf32, accum, 0);
    if (rc) return rc;
  }
  return 0;
}

/*
 * Fast contiguous fp32-accumulating variant, kept as an extra CPU timing: C = A @ B with A [m,k],
 * B [k,n] row-major 16-bit operands.  Each output is the float32 running sum over k in index
 * order, so it is bit-equal to oracle_gemm with ORACLE_ACCUM_F32 (pinned in tests/test_oracle.py).  Work is split into (16-row x 256-column) blocks over
 * OpenMP threads; each block keeps its fp32 accumulators in L1 and streams the matching B
 * column panel once per block, converting 16-bit values as it goes.  scratch_rows is unused
 * (kept for ABI stability of the test binding).
 */
#define FAST_RB 16
#define FAST_NB 256
int oracle_gemm_rowmajor_fast(const uint16_t* a, const uint16_t* b, uint16_t* c, int32_t m, int32_t n, int32_t k,
                              int32_t dtype, float* scratch_rows, int32_t threads) {
  if (dtype != ORACLE_F16 && dtype != ORACLE_BF16) return -1;
  (void)scratch_rows;
  const int32_t row_blocks = (m + FAST_RB - 1) / FAST_RB;
  const int32_t col_blocks = (n + FAST_NB - 1) / FAST_NB;
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads) collapse(2)
  for (int32_t rb = 0; rb < row_blocks; ++rb) {
    for (int32_t cb = 0; cb < col_blocks; ++cb) {
      float acc[FAST_RB][FAST_NB];
      float bconv[FAST_NB];
      const int32_t r0 = rb * FAST_RB, c0 = cb * FAST_NB;
      const int32_t rows = (m - r0) < FAST_RB ? (m - r0) : FAST_RB;
      const int32_t cols = (n - c0) < FAST_NB ? (n - c0) : FAST_NB;
      for (int32_t r = 0; r < FAST_RB; ++r)
        for (int32_t j = 0; j < FAST_NB; ++j) acc[r][j] = 0.0f;
      for (int32_t l = 0; l < k; ++l) {
        const uint16_t* brow = b + (int64_t)l * n + c0;
        if (dtype == ORACLE_BF16) {
          for (int32_t j = 0; j < cols; ++j) bconv[j] = bits_to_float((uint32_t)brow[j] << 16);
        } else {
          for (int32_t j = 0; j < cols; ++j) bconv[j] = oracle_f16_to_float(brow[j]);
        }
        for (int32_t r = 0; r < rows; ++r) {
          const uint16_t av = a[(int64_t)(r0 + r) * k + l];
          const float x = dtype == ORACLE_BF16 ? oracle_bf16_to_float(av) : oracle_f16_to_float(av);
          for (int32_t j = 0; j < cols; ++j) acc[r][j] += x * bconv[j];
        }
      }
      for (int32_t r = 0; r < rows; ++r)
        for (int32_t j = 0; j < cols; ++j)
          c[(int64_t)(r0 + r) * n + c0 + j] =
              dtype == ORACLE_BF16 ? oracle_float_to_bf16(acc[r][j]) : oracle_float_to_f16(acc[r][j]);
    }
  }
  return 0;
}

/*
 * csr_oracle.c - TEST INFRASTRUCTURE ONLY.
 *
 * Plain-C restatement of mlx-sparse's CPU CSR sparse x dense kernels, used
 * as the parity checker for the HIP library and as the CPU baseline that
 * bench.py times.  Nothing in the product links or calls this file; only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 *
 * What it restates (reference files under mlx-sparse):
 *   - per-row SpMV sum, stored order, lengths 0..4 written out in the same
 *     left-to-right order (src/sparse/csr_matvec/csr_matvec.cpp:79-114);
 *   - the SpMV driver: serial O(n) row-work prepass, work-balanced row
 *     ranges, one std::thread per extra range, spawned per call
 *     (csr_matvec.cpp:116-168, src/common/cpu_parallel.h:50-97);
 *   - SpMM: one accumulator per RHS column, rows summed in stored order,
 *     row work nnz_row * k (src/sparse/csr_matmul/csr_matmul.cpp:83-222);
 *   - accumulator rules: float32 -> float32, complex64 -> complex64,
 *     float16/bfloat16 -> float32 with operands widened before the multiply
 *     and one rounding at the end (src/common/common.h:52-79);
 *   - worker-count resolution and range partitioning
 *     (src/common/cpu_parallel.cpp:46-253, cpu_parallel.h:134-164);
 *   - the adjoint side: the CSR transpose by counting sort
 *     (src/sparse/csr_transpose/csr_transpose.cpp, csr_transpose_cpu_impl),
 *     the transposed products with their per-range partial outputs added in
 *     range order (src/sparse/csr_matvec_transpose/csr_matvec_transpose.cpp,
 *     csr_matmul_transpose/csr_matmul_transpose.cpp, *_cpu_impl) and the
 *     value gradients (csr_matvec_data_vjp.cpp, csr_matmul_data_vjp.cpp);
 *   - the conjugate gradient solver (src/linalg/cg/cg.cpp:75-246,
 *     csr_cg_cpu_impl) with its float SpMV summed from zero
 *     (src/linalg/common/common.h:35-45, csr_spmv_float), and the
 *     Jacobi-preconditioned CG (src/preconditioners/pcg/pcg.cpp:71-236,
 *     csr_pcg_jacobi_cpu_impl), float32 values only;
 *   - BiCGSTAB (src/linalg/bicgstab/bicgstab.cpp:80-362, csr_bicgstab_cpu_impl)
 *     and MINRES with its shift (src/linalg/minres/minres.cpp:68-312,
 *     csr_minres_cpu_impl), float32;
 *   - BiCGSTAB, MINRES and restarted GMRES with a Jacobi preconditioner
 *     (src/preconditioners/bicgstab/bicgstab.cpp:140-521,
 *     src/preconditioners/minres/minres.cpp:93-330,
 *     src/preconditioners/gmres/gmres.cpp:342-748), float32;
 *   - restarted GMRES (src/linalg/gmres/gmres.cpp:58-220, csr_gmres_impl)
 *     with its Arnoldi factorisation (src/linalg/arnoldi/arnoldi.cpp:79-159,
 *     csr_arnoldi_cpu_impl) and the Givens least-squares solve
 *     (src/linalg/common/common.h:143-234), float32.
 *
 * Built with -ffp-contract=off so every product and every sum is rounded on
 * its own, as the reference's separate multiply_accumulate / `+=` are.
 *
 * Pinning (tests/test_oracle_*.py): reference KATs and SciPy products,
 * SuiteSparse fixtures, closed forms of stencil matrices, float64 brute
 * force on small inputs, numpy's float16 rounding and an exhaustive check of
 * the bfloat16 rounding rule, and a naive re-derivation of the range rule.
 * The exact float16/bfloat16 rounding and complex product of MLX
 * (mx::float16_t, mx::bfloat16_t, mx::complex64_t, un-vendored) are assumed
 * IEEE round-to-nearest-even and textbook; only tolerance tests pin them.
 */
#define _GNU_SOURCE
#include <errno.h>
#include <float.h>
#include <limits.h>
#include <math.h>
#include <pthread.h>
#include <sched.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

enum { V_F32 = 0, V_F16 = 1, V_BF16 = 2, V_C64 = 3 };
enum { I_I32 = 0, I_I64 = 1 };

typedef struct {
  float re, im;
} cf32;

/* ---------------------------------------------------------------------- */
/* float16 / bfloat16 <-> float32, from the IEEE 754 binary16 layout and the
 * bfloat16 layout (top 16 bits of binary32).  Narrowing rounds to nearest,
 * ties to even. */

static float f32_from_bits(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static uint32_t bits_from_f32(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

float oracle_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  if (exp == 0) {
    if (man == 0) return f32_from_bits(sign);
    /* subnormal: value = man * 2^-24, exact in binary32 */
    float v = (float)man * 5.9604644775390625e-8f;
    return sign ? -v : v;
  }
  if (exp == 31) return f32_from_bits(sign | 0x7f800000u | (man << 13));
  return f32_from_bits(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t oracle_f32_to_f16(float f) {
  uint32_t u = bits_from_f32(f);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu)); /* NaN */
  if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to inf */
  if (a < 0x38800000u) {
    /* result is subnormal or zero: scale to units of 2^-24 and round */
    int e = (int)(a >> 23);                       /* biased binary32 exponent */
    if (e < 102) return sign;                     /* below half of 2^-24 */
    uint32_t m = (a & 0x7fffffu) | 0x800000u;     /* 24-bit significand */
    int shift = 126 - e;                          /* (e-127)-23+24 => right shift */
    uint32_t q = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
  }
  /* normal: rebias exponent, round 13 dropped bits to nearest even */
  uint32_t r = a - 0x38000000u; /* exponent 127 -> 15 */
  uint32_t q = r >> 13;
  uint32_t rem = r & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
  return (uint16_t)(sign | q);
}

float oracle_bf16_to_f32(uint16_t b) { return f32_from_bits((uint32_t)b << 16); }

uint16_t oracle_f32_to_bf16(float f) {
  uint32_t u = bits_from_f32(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u); /* quiet NaN */
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return (uint16_t)(u >> 16);
}

/* ---------------------------------------------------------------------- */
/* Accumulator rules (reference: src/common/common.h:52-79). */

static inline float mul_f32(float a, float b) { return a * b; }
static inline cf32 mul_c64(cf32 a, cf32 b) {
  float rr = a.re * b.re;
  float ii = a.im * b.im;
  float ri = a.re * b.im;
  float ir = a.im * b.re;
  cf32 r = {rr - ii, ri + ir};
  return r;
}
static inline cf32 add_c64(cf32 a, cf32 b) {
  cf32 r = {a.re + b.re, a.im + b.im};
  return r;
}

static inline float widen(int vt, const void *base, int64_t i) {
  switch (vt) {
  case V_F16: return oracle_f16_to_f32(((const uint16_t *)base)[i]);
  case V_BF16: return oracle_bf16_to_f32(((const uint16_t *)base)[i]);
  default: return ((const float *)base)[i];
  }
}

static inline void narrow_store(int vt, void *base, int64_t i, float v) {
  switch (vt) {
  case V_F16: ((uint16_t *)base)[i] = oracle_f32_to_f16(v); break;
  case V_BF16: ((uint16_t *)base)[i] = oracle_f32_to_bf16(v); break;
  default: ((float *)base)[i] = v; break;
  }
}

static inline int64_t load_index(int it, const void *base, int64_t i) {
  return it == I_I64 ? ((const int64_t *)base)[i] : (int64_t)((const int32_t *)base)[i];
}

/* One SpMV row: restates csr_matvec_row_accum (csr_matvec.cpp:79-114).
 * Lengths 1..4 start from the first product (no leading +0.0), longer rows
 * start from the zero accumulator, both summed left to right. */
static void matvec_row(int vt, int it, const void *data, const void *indices,
                       int64_t begin, int64_t end, const void *x, void *y,
                       int64_t row) {
  int64_t len = end - begin;
  if (vt == V_C64) {
    const cf32 *d = (const cf32 *)data, *xv = (const cf32 *)x;
    cf32 acc = {0.0f, 0.0f};
    int64_t p = begin;
    if (len >= 1 && len <= 4) {
      acc = mul_c64(d[p], xv[load_index(it, indices, p)]);
      p++;
    }
    for (; p < end; ++p) acc = add_c64(acc, mul_c64(d[p], xv[load_index(it, indices, p)]));
    ((cf32 *)y)[row] = acc;
    return;
  }
  float acc = 0.0f;
  int64_t p = begin;
  if (len >= 1 && len <= 4) {
    acc = mul_f32(widen(vt, data, p), widen(vt, x, load_index(it, indices, p)));
    p++;
  }
  for (; p < end; ++p)
    acc = acc + mul_f32(widen(vt, data, p), widen(vt, x, load_index(it, indices, p)));
  narrow_store(vt, y, row, acc);
}

/* SpMM rows [r0, r1): restates csr_matmul_small_rhs_cpu_impl and
 * csr_matmul_generic_cpu_impl (csr_matmul.cpp:83-133); both sum each column
 * from the zero accumulator in stored order. */
static void matmul_rows(int vt, int it, const void *data, const void *indices,
                        const void *indptr, const void *X, void *Y, int64_t k,
                        int64_t r0, int64_t r1, void *scratch) {
  for (int64_t row = r0; row < r1; ++row) {
    int64_t b = load_index(it, indptr, row), e = load_index(it, indptr, row + 1);
    if (vt == V_C64) {
      cf32 *acc = (cf32 *)scratch;
      for (int64_t c = 0; c < k; ++c) acc[c].re = acc[c].im = 0.0f;
      const cf32 *d = (const cf32 *)data, *xv = (const cf32 *)X;
      for (int64_t p = b; p < e; ++p) {
        const cf32 *xr = xv + load_index(it, indices, p) * k;
        for (int64_t c = 0; c < k; ++c) acc[c] = add_c64(acc[c], mul_c64(d[p], xr[c]));
      }
      for (int64_t c = 0; c < k; ++c) ((cf32 *)Y)[row * k + c] = acc[c];
    } else {
      float *acc = (float *)scratch;
      for (int64_t c = 0; c < k; ++c) acc[c] = 0.0f;
      for (int64_t p = b; p < e; ++p) {
        float v = widen(vt, data, p);
        int64_t off = load_index(it, indices, p) * k;
        for (int64_t c = 0; c < k; ++c) acc[c] = acc[c] + mul_f32(v, widen(vt, X, off + c));
      }
      for (int64_t c = 0; c < k; ++c) narrow_store(vt, Y, row * k + c, acc[c]);
    }
  }
}

/* ---------------------------------------------------------------------- */
/* Worker count and ranges (reference: src/common/cpu_parallel.cpp:46-253). */

static int parse_positive_int(const char *v) {
  if (v == NULL || *v == '\0') return 0;
  char *end = NULL;
  errno = 0;
  long parsed = strtol(v, &end, 10);
  if (end == v || parsed <= 0 || parsed > INT_MAX) return 0;
  if (*end != '\0' && *end != ',') return 0;
  return (int)parsed;
}

int oracle_cpu_worker_count(void) {
  const char *raw = getenv("MLX_SPARSE_CPU_THREADS");
  if (raw == NULL || *raw == '\0') raw = getenv("MLX_SPARSE_N_THREADS");
  int c = parse_positive_int(raw);
  if (c > 0) return c;
  c = parse_positive_int(getenv("OMP_NUM_THREADS"));
  if (c > 0) return c;
  const char *names[] = {"SLURM_CPUS_PER_TASK", "PBS_NP", "LSB_DJOB_NUMPROC", "NSLOTS"};
  for (int i = 0; i < 4; ++i) {
    c = parse_positive_int(getenv(names[i]));
    if (c > 0) return c;
  }
  cpu_set_t set;
  CPU_ZERO(&set);
  if (sched_getaffinity(0, sizeof(set), &set) == 0) {
    c = CPU_COUNT(&set);
    if (c > 0) return c;
  }
  long hw = sysconf(_SC_NPROCESSORS_ONLN);
  return hw > 0 ? (int)hw : 1;
}

/* equal_cpu_ranges: part p gets [p*n/count, (p+1)*n/count), empties dropped. */
static int64_t equal_ranges(int64_t n, int parts, int64_t *out) {
  if (n <= 0) return 0;
  int count = parts < 1 ? 1 : parts;
  int64_t m = 0;
  for (int p = 0; p < count; ++p) {
    int64_t b = ((int64_t)p * n) / count, e = ((int64_t)(p + 1) * n) / count;
    if (b < e) {
      out[2 * m] = b;
      out[2 * m + 1] = e;
      m++;
    }
  }
  return m;
}

/* weighted_cpu_ranges: walk the work prefix sum, each part takes rows up to
 * the first prefix >= begin_prefix + ceil(remaining / remaining_parts),
 * at least one row, leaving one row for each later part. */
static int64_t weighted_ranges(const int64_t *work, int64_t n, int parts, int64_t *out) {
  if (n <= 0) return 0;
  int count = parts < 1 ? 1 : parts;
  if (count == 1) {
    out[0] = 0;
    out[1] = n;
    return 1;
  }
  if (count >= n) return equal_ranges(n, count, out);
  int64_t *prefix = (int64_t *)malloc((size_t)(n + 1) * sizeof(int64_t));
  if (!prefix) return -1;
  prefix[0] = 0;
  for (int64_t r = 0; r < n; ++r) {
    int64_t w = work[r] > 0 ? work[r] : 0;
    int64_t next = prefix[r] + w;
    prefix[r + 1] = next < prefix[r] ? INT64_MAX : next;
  }
  if (prefix[n] <= 0) {
    free(prefix);
    return equal_ranges(n, count, out);
  }
  int64_t m = 0, begin = 0;
  for (int part = 0; part < count && begin < n; ++part) {
    int remaining_parts = count - part;
    if (remaining_parts == 1) {
      out[2 * m] = begin;
      out[2 * m + 1] = n;
      m++;
      break;
    }
    int64_t remaining = prefix[n] - prefix[begin];
    int64_t target = prefix[begin] + (remaining + remaining_parts - 1) / remaining_parts;
    /* lower_bound over prefix[begin+1 .. n] */
    int64_t lo = begin + 1, hi = n + 1;
    while (lo < hi) {
      int64_t mid = lo + (hi - lo) / 2;
      if (prefix[mid] < target) lo = mid + 1;
      else hi = mid;
    }
    int64_t end = lo;
    if (end < begin + 1) end = begin + 1;
    if (end > n - (remaining_parts - 1)) end = n - (remaining_parts - 1);
    out[2 * m] = begin;
    out[2 * m + 1] = end;
    m++;
    begin = end;
  }
  free(prefix);
  return m;
}

/* cpu_ranges_for_output_work (cpu_parallel.h:134-164). Returns the number of
 * ranges written into out (2 * parts capacity), or -1 on allocation failure. */
int64_t oracle_cpu_ranges(const int64_t *work, int64_t n, int parts, int64_t *out) {
  if (n <= 0) return 0;
  if (parts <= 1) {
    out[0] = 0;
    out[1] = n;
    return 1;
  }
  int imbalance = 0;
  int64_t prev = -1;
  for (int64_t i = 0; i < n; ++i) {
    int64_t c = work[i] > 0 ? work[i] : 0;
    if (prev >= 0 && c != prev) {
      imbalance = 1;
      break;
    }
    prev = c;
  }
  if (!imbalance) return equal_ranges(n, parts, out);
  return weighted_ranges(work, n, parts, out);
}

/* ---------------------------------------------------------------------- */
/* Drivers. */

typedef struct {
  int op; /* 0 = matvec, 1 = matmul */
  int vt, it;
  const void *data, *indices, *indptr, *x;
  void *y;
  int64_t k;
  int64_t r0, r1;
  int failed;
} job_t;

static void run_job(job_t *j) {
  if (j->op == 0) {
    for (int64_t r = j->r0; r < j->r1; ++r)
      matvec_row(j->vt, j->it, j->data, j->indices, load_index(j->it, j->indptr, r),
                 load_index(j->it, j->indptr, r + 1), j->x, j->y, r);
  } else {
    size_t bytes = (size_t)(j->k > 0 ? j->k : 1) * (j->vt == V_C64 ? 8 : 4);
    void *scratch = malloc(bytes);
    if (!scratch) {
      j->failed = 1;
      return;
    }
    matmul_rows(j->vt, j->it, j->data, j->indices, j->indptr, j->x, j->y, j->k, j->r0, j->r1,
                scratch);
    free(scratch);
  }
}

static void *job_thread(void *arg) {
  run_job((job_t *)arg);
  return NULL;
}

/* Shared driver: n_threads <= 0 resolves the worker count like the
 * reference.  Returns 0 on success. */
static int drive(job_t base, int64_t n_rows, int n_threads) {
  int workers = n_threads > 0 ? n_threads : oracle_cpu_worker_count();
  if (workers <= 1 || n_rows <= 0) {
    base.r0 = 0;
    base.r1 = n_rows;
    run_job(&base);
    return base.failed ? -1 : 0;
  }
  int64_t *work = (int64_t *)malloc((size_t)n_rows * sizeof(int64_t));
  int64_t *ranges = (int64_t *)malloc((size_t)workers * 2 * sizeof(int64_t));
  if (!work || !ranges) {
    free(work);
    free(ranges);
    return -1;
  }
  int64_t kk = base.op == 1 ? (base.k > 1 ? base.k : 1) : 1;
  for (int64_t r = 0; r < n_rows; ++r)
    work[r] = (load_index(base.it, base.indptr, r + 1) - load_index(base.it, base.indptr, r)) * kk;
  int64_t m = oracle_cpu_ranges(work, n_rows, workers, ranges);
  free(work);
  if (m < 0) {
    free(ranges);
    return -1;
  }
  if (m <= 1) {
    free(ranges);
    base.r0 = 0;
    base.r1 = n_rows;
    run_job(&base);
    return base.failed ? -1 : 0;
  }
  job_t *jobs = (job_t *)calloc((size_t)m, sizeof(job_t));
  pthread_t *th = (pthread_t *)calloc((size_t)m, sizeof(pthread_t));
  if (!jobs || !th) {
    free(jobs);
    free(th);
    free(ranges);
    return -1;
  }
  for (int64_t i = 0; i < m; ++i) {
    jobs[i] = base;
    jobs[i].r0 = ranges[2 * i];
    jobs[i].r1 = ranges[2 * i + 1];
  }
  int rc = 0;
  int64_t started = 1;
  for (int64_t i = 1; i < m; ++i) {
    if (pthread_create(&th[i], NULL, job_thread, &jobs[i]) != 0) {
      jobs[i].failed = 1;
      break;
    }
    started++;
  }
  run_job(&jobs[0]);
  for (int64_t i = 1; i < started; ++i) pthread_join(th[i], NULL);
  for (int64_t i = 0; i < m; ++i)
    if (jobs[i].failed) rc = -1;
  free(jobs);
  free(th);
  free(ranges);
  return rc;
}

int oracle_csr_matvec(int vt, int it, int64_t n_rows, const void *data, const void *indices,
                      const void *indptr, const void *x, void *y, int n_threads) {
  job_t j;
  memset(&j, 0, sizeof(j));
  j.op = 0;
  j.vt = vt;
  j.it = it;
  j.data = data;
  j.indices = indices;
  j.indptr = indptr;
  j.x = x;
  j.y = y;
  return drive(j, n_rows, n_threads);
}

int oracle_csr_matmul(int vt, int it, int64_t n_rows, int64_t k, const void *data,
                      const void *indices, const void *indptr, const void *X, void *Y,
                      int n_threads) {
  job_t j;
  memset(&j, 0, sizeof(j));
  j.op = 1;
  j.vt = vt;
  j.it = it;
  j.data = data;
  j.indices = indices;
  j.indptr = indptr;
  j.x = X;
  j.y = Y;
  j.k = k;
  return drive(j, n_rows, n_threads);
}

/* Array forms of the conversions, for tests that pin them. kind: 0 = f16,
 * 1 = bf16. */
void oracle_narrow_array(int kind, const float *src, uint16_t *dst, int64_t n) {
  for (int64_t i = 0; i < n; ++i)
    dst[i] = kind == 0 ? oracle_f32_to_f16(src[i]) : oracle_f32_to_bf16(src[i]);
}

void oracle_widen_array(int kind, const uint16_t *src, float *dst, int64_t n) {
  for (int64_t i = 0; i < n; ++i)
    dst[i] = kind == 0 ? oracle_f16_to_f32(src[i]) : oracle_bf16_to_f32(src[i]);
}

/* ---------------------------------------------------------------------- */
/* Adjoint side.  Accumulators as above; columns outside [0, n_cols) are
 * skipped (the reference indexes with them unchecked). */

static inline int col_ok(int64_t c, int64_t n_cols) { return c >= 0 && c < n_cols; }

/* Rows [r0, r1) of A^T X added into acc (n_cols * k, float or cf32). */
static void transpose_rows(int vt, int it, const void *data, const void *indices, const void *indptr,
                           const void *X, int64_t n_cols, int64_t k, int64_t r0, int64_t r1,
                           void *acc) {
  for (int64_t r = r0; r < r1; ++r) {
    int64_t b = load_index(it, indptr, r), e = load_index(it, indptr, r + 1);
    for (int64_t p = b; p < e; ++p) {
      int64_t c = load_index(it, indices, p);
      if (!col_ok(c, n_cols)) continue;
      for (int64_t q = 0; q < k; ++q) {
        if (vt == V_C64) {
          cf32 *a = (cf32 *)acc + c * k + q;
          *a = add_c64(*a, mul_c64(((const cf32 *)data)[p], ((const cf32 *)X)[r * k + q]));
        } else {
          float *a = (float *)acc + c * k + q;
          *a = *a + mul_f32(widen(vt, data, p), widen(vt, X, r * k + q));
        }
      }
    }
  }
}

/* A^T X (k = 1: A^T x).  One worker: every output from zero over the rows
 * in order.  W workers: the rows split by row length (the SpMV ranges),
 * each range's partial output from zero, partials added from zero in range
 * order.  Returns 0 on success. */
int oracle_csr_transpose_product(int vt, int it, int64_t n_rows, int64_t n_cols, int64_t k,
                                 const void *data, const void *indices, const void *indptr,
                                 const void *X, void *Y, int n_threads) {
  int workers = n_threads > 0 ? n_threads : oracle_cpu_worker_count();
  int64_t out = n_cols * k;
  size_t esz = vt == V_C64 ? sizeof(cf32) : sizeof(float);
  int64_t m = 1;
  int64_t *ranges = NULL;
  if (workers > 1 && n_rows > 0 && out > 0) {
    int64_t *work = (int64_t *)malloc((size_t)n_rows * sizeof(int64_t));
    ranges = (int64_t *)malloc((size_t)workers * 2 * sizeof(int64_t));
    if (!work || !ranges) {
      free(work);
      free(ranges);
      return -1;
    }
    for (int64_t r = 0; r < n_rows; ++r)
      work[r] = load_index(it, indptr, r + 1) - load_index(it, indptr, r);
    m = oracle_cpu_ranges(work, n_rows, workers, ranges);
    free(work);
    if (m < 1) m = 1;
  }
  void *partial = calloc((size_t)(m * (out > 0 ? out : 1)), esz);
  if (!partial) {
    free(ranges);
    return -1;
  }
  if (m <= 1) {
    transpose_rows(vt, it, data, indices, indptr, X, n_cols, k, 0, n_rows, partial);
  } else {
    for (int64_t w = 0; w < m; ++w)
      transpose_rows(vt, it, data, indices, indptr, X, n_cols, k, ranges[2 * w], ranges[2 * w + 1],
                     (char *)partial + (size_t)(w * out) * esz);
  }
  for (int64_t i = 0; i < out; ++i) {
    if (vt == V_C64) {
      cf32 t = {0.0f, 0.0f};
      if (m <= 1) t = ((cf32 *)partial)[i];
      else
        for (int64_t w = 0; w < m; ++w) t = add_c64(t, ((cf32 *)partial)[w * out + i]);
      ((cf32 *)Y)[i] = t;
    } else {
      float t = 0.0f;
      if (m <= 1) t = ((float *)partial)[i];
      else
        for (int64_t w = 0; w < m; ++w) t = t + ((float *)partial)[w * out + i];
      narrow_store(vt, Y, i, t);
    }
  }
  free(partial);
  free(ranges);
  return 0;
}

/* CSR of A^T: column counts, prefix sums, then rows in order. */
int oracle_csr_transpose(int vt, int it, int64_t n_rows, int64_t n_cols, const void *data,
                         const void *indices, const void *indptr, void *t_data, void *t_indices,
                         void *t_indptr) {
  size_t esz = vt == V_C64 ? 8 : (vt == V_F32 ? 4 : 2);
  int64_t *next = (int64_t *)calloc((size_t)n_cols + 1, sizeof(int64_t));
  if (!next) return -1;
  for (int64_t r = 0; r < n_rows; ++r)
    for (int64_t p = load_index(it, indptr, r); p < load_index(it, indptr, r + 1); ++p) {
      int64_t c = load_index(it, indices, p);
      if (col_ok(c, n_cols)) next[c + 1]++;
    }
  for (int64_t c = 0; c < n_cols; ++c) next[c + 1] += next[c];
  for (int64_t c = 0; c <= n_cols; ++c) {
    if (it == I_I64) ((int64_t *)t_indptr)[c] = next[c];
    else ((int32_t *)t_indptr)[c] = (int32_t)next[c];
  }
  for (int64_t r = 0; r < n_rows; ++r)
    for (int64_t p = load_index(it, indptr, r); p < load_index(it, indptr, r + 1); ++p) {
      int64_t c = load_index(it, indices, p);
      if (!col_ok(c, n_cols)) continue;
      int64_t slot = next[c]++;
      memcpy((char *)t_data + (size_t)slot * esz, (const char *)data + (size_t)p * esz, esz);
      if (it == I_I64) ((int64_t *)t_indices)[slot] = r;
      else ((int32_t *)t_indices)[slot] = (int32_t)r;
    }
  free(next);
  return 0;
}

/* Value gradients.  single != 0: out[p] = cot[row] * x[col] (one product,
 * the SpMV rule); else out[p] = sum_q cot[row, q] * X[col, q] from zero. */
int oracle_csr_data_vjp(int vt, int it, int64_t n_rows, int64_t n_cols, int64_t k, int single,
                        const void *indices, const void *indptr, const void *X, const void *cot,
                        void *out) {
  for (int64_t r = 0; r < n_rows; ++r)
    for (int64_t p = load_index(it, indptr, r); p < load_index(it, indptr, r + 1); ++p) {
      int64_t c = load_index(it, indices, p);
      if (vt == V_C64) {
        cf32 acc = {0.0f, 0.0f};
        if (col_ok(c, n_cols)) {
          if (single) acc = mul_c64(((const cf32 *)cot)[r], ((const cf32 *)X)[c]);
          else
            for (int64_t q = 0; q < k; ++q)
              acc = add_c64(acc, mul_c64(((const cf32 *)cot)[r * k + q], ((const cf32 *)X)[c * k + q]));
        }
        ((cf32 *)out)[p] = acc;
      } else {
        float acc = 0.0f;
        if (col_ok(c, n_cols)) {
          if (single) acc = mul_f32(widen(vt, cot, r), widen(vt, X, c));
          else
            for (int64_t q = 0; q < k; ++q)
              acc = acc + mul_f32(widen(vt, cot, r * k + q), widen(vt, X, c * k + q));
        }
        narrow_store(vt, out, p, acc);
      }
    }
  return 0;
}

/* ---------------------------------------------------------------------- */
/* Krylov solvers (float32).  The solver SpMV sums each row from 0.0f in
 * stored order; scalars and dot products are double unless noted. */

static void cg_spmv(int it, int64_t n, const float *data, const void *indices, const void *indptr,
                    const float *x, float *out) {
  for (int64_t r = 0; r < n; ++r) {
    float acc = 0.0f;
    for (int64_t p = load_index(it, indptr, r); p < load_index(it, indptr, r + 1); ++p) {
      const int64_t c = load_index(it, indices, p);
      if (c >= 0 && c < n) acc = acc + data[p] * x[c];
    }
    out[r] = acc;
  }
}

static int fin(float v) { return isfinite(v); }

/* std::max(v, 0) of the reference: a NaN stays NaN. */
static double max0(double v) { return v < 0.0 ? 0.0 : v; }
static float max0f(float v) { return v < 0.0f ? 0.0f : v; }

/* Conjugate gradients: x from x0; info 0 converged, maxiter (or 1 when
 * maxiter is 0) when the budget ran out, -1 near-zero denominator, -3
 * non-finite.  residual = float(sqrt(r.r)), iterations = completed steps. */
int oracle_csr_cg(int it, int64_t n, const float *data, const void *indices, const void *indptr,
                  const float *b, const float *x0, float *x, float rtol, float atol,
                  int64_t maxiter, int32_t *info, float *residual, int32_t *iterations) {
  float *r = (float *)malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
  float *p = (float *)malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
  float *ap = (float *)malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
  if (!r || !p || !ap) {
    free(r);
    free(p);
    free(ap);
    return -1;
  }
  memcpy(x, x0, (size_t)n * sizeof(float));
  cg_spmv(it, n, data, indices, indptr, x, ap);
  double b_norm2 = 0.0, rr = 0.0;
  int finite = 1;
  for (int64_t i = 0; i < n; ++i) {
    r[i] = b[i] - ap[i];
    p[i] = r[i];
    b_norm2 += (double)b[i] * (double)b[i];
    rr += (double)r[i] * (double)r[i];
    finite = finite && fin(r[i]) && fin(p[i]) && fin(ap[i]) && fin(b[i]) && fin(x[i]);
  }
  const float residual_norm = (float)sqrt(max0(rr));
  const float b_norm = (float)sqrt(max0(b_norm2));
  const float scaled = rtol * b_norm;
  const float tol = atol > scaled ? atol : scaled;
  const float eps = FLT_EPSILON;
  int32_t status;
  int32_t completed = 0;
  if (!finite || !isfinite(rr) || !fin(residual_norm) || !fin(b_norm)) {
    *info = -3;
    *residual = residual_norm;
    *iterations = 0;
    goto done;
  }
  if (residual_norm <= tol) {
    *info = 0;
    *residual = residual_norm;
    *iterations = 0;
    goto done;
  }
  status = maxiter > 0 ? (int32_t)maxiter : 1;
  for (int64_t k = 1; k <= maxiter; ++k) {
    cg_spmv(it, n, data, indices, indptr, p, ap);
    double denom = 0.0;
    finite = 1;
    for (int64_t i = 0; i < n; ++i) {
      denom += (double)p[i] * (double)ap[i];
      finite = finite && fin(p[i]) && fin(ap[i]);
    }
    if (!finite || !isfinite(denom)) {
      status = -3;
      completed = (int32_t)(k - 1);
      break;
    }
    if (fabs(denom) <= (double)eps) {
      double p2 = 0.0, ap2 = 0.0;
      for (int64_t i = 0; i < n; ++i) {
        p2 += (double)p[i] * (double)p[i];
        ap2 += (double)ap[i] * (double)ap[i];
      }
      const double prod = p2 * ap2;
      const double scale = sqrt(max0(prod));
      const double grown = (double)eps * (double)eps * (scale > 1.0 ? scale : 1.0);
      const double dtol = (double)eps < grown ? (double)eps : grown;
      if (!isfinite(scale)) {
        status = -3;
        completed = (int32_t)(k - 1);
        break;
      }
      if (fabs(denom) <= dtol) {
        status = -1;
        completed = (int32_t)(k - 1);
        break;
      }
    }
    const double alpha = rr / denom;
    if (!isfinite(alpha)) {
      status = -3;
      completed = (int32_t)(k - 1);
      break;
    }
    finite = 1;
    double rr_new = 0.0;
    for (int64_t i = 0; i < n; ++i) {
      const double xc = (double)x[i] + alpha * (double)p[i];
      const double rc = (double)r[i] - alpha * (double)ap[i];
      const float xf = (float)xc, rf = (float)rc;
      if (!isfinite(xc) || !isfinite(rc) || !fin(xf) || !fin(rf)) {
        finite = 0;
        continue;
      }
      x[i] = xf;
      r[i] = rf;
      rr_new += (double)rf * (double)rf;
    }
    const float r_norm = (float)sqrt(max0(rr_new));
    completed = (int32_t)k;
    if (!finite || !isfinite(rr_new) || !fin(r_norm)) {
      status = -3;
      break;
    }
    if (r_norm <= tol) {
      status = 0;
      rr = rr_new;
      break;
    }
    const double beta = rr_new / rr;
    if (!isfinite(beta)) {
      status = -3;
      break;
    }
    for (int64_t i = 0; i < n; ++i) {
      const double pc = (double)r[i] + beta * (double)p[i];
      const float pf = (float)pc;
      if (!isfinite(pc) || !fin(pf)) {
        status = -3;
        break;
      }
      p[i] = pf;
    }
    if (status < 0) break;
    rr = rr_new;
  }
  *info = status;
  *residual = (float)sqrt(max0(rr));
  *iterations = completed;
done:
  free(r);
  free(p);
  free(ap);
  return 0;
}

static float dot_f(const float *a, const float *b, int64_t n) {
  double acc = 0.0;
  for (int64_t i = 0; i < n; ++i) acc += (double)a[i] * (double)b[i];
  return (float)acc;
}

/* Jacobi-preconditioned CG (z = inv_diag * r): float scalars from double
 * sums, float vector updates; info -2 for a non-positive r.z. */
int oracle_csr_pcg_jacobi(int it, int64_t n, const float *data, const void *indices,
                          const void *indptr, const float *b, const float *x0,
                          const float *inv_diag, float *x, float rtol, float atol,
                          int64_t maxiter, int32_t *info, float *residual, int32_t *iterations) {
  const size_t bytes = (size_t)(n > 0 ? n : 1) * sizeof(float);
  float *r = (float *)malloc(bytes), *z = (float *)malloc(bytes), *p = (float *)malloc(bytes);
  float *ap = (float *)malloc(bytes);
  if (!r || !z || !p || !ap) {
    free(r);
    free(z);
    free(p);
    free(ap);
    return -1;
  }
  memcpy(x, x0, (size_t)n * sizeof(float));
  cg_spmv(it, n, data, indices, indptr, x, ap);
  double b_norm2 = 0.0;
  int finite = 1;
  for (int64_t i = 0; i < n; ++i) {
    const float ri = b[i] - ap[i];
    const float zi = inv_diag[i] * ri;
    r[i] = ri;
    z[i] = zi;
    p[i] = zi;
    b_norm2 += (double)b[i] * (double)b[i];
    finite = finite && fin(ri) && fin(zi) && fin(inv_diag[i]);
  }
  float true_rr = dot_f(r, r, n);
  float rho = dot_f(r, z, n);
  const float b_norm = (float)sqrt(max0(b_norm2));
  const float scaled = rtol * b_norm;
  const float tol = atol > scaled ? atol : scaled;
  const float true_residual = sqrtf(max0f(true_rr));
  const float eps = FLT_EPSILON;
  int32_t status, completed = 0;
  if (!finite || !fin(true_rr) || !fin(rho)) {
    *info = -3;
    *residual = true_residual;
    *iterations = 0;
    goto done;
  }
  if (true_residual <= tol) {
    *info = 0;
    *residual = true_residual;
    *iterations = 0;
    goto done;
  }
  if (rho <= 0.0f) {
    *info = -2;
    *residual = true_residual;
    *iterations = 0;
    goto done;
  }
  status = maxiter > 0 ? (int32_t)maxiter : 1;
  for (int64_t k = 1; k <= maxiter; ++k) {
    cg_spmv(it, n, data, indices, indptr, p, ap);
    const float denom = dot_f(p, ap, n);
    const float p2 = dot_f(p, p, n);
    const float ap2 = dot_f(ap, ap, n);
    const float prod = p2 * ap2;
    const float scale = sqrtf(max0f(prod));
    const float dtol = eps * (scale > 1.0f ? scale : 1.0f);
    if (!fin(denom) || !fin(scale) || fabsf(denom) <= dtol) {
      status = -1;
      completed = (int32_t)(k - 1);
      break;
    }
    const float alpha = rho / denom;
    if (!fin(alpha)) {
      status = -3;
      completed = (int32_t)(k - 1);
      break;
    }
    double acc = 0.0;
    finite = 1;
    for (int64_t i = 0; i < n; ++i) {
      x[i] = x[i] + alpha * p[i];
      const float ri = r[i] - alpha * ap[i];
      const float zi = inv_diag[i] * ri;
      r[i] = ri;
      z[i] = zi;
      acc += (double)ri * (double)ri;
      finite = finite && fin(x[i]) && fin(ri) && fin(zi);
    }
    true_rr = (float)acc;
    const float r_norm = sqrtf(max0f(true_rr));
    completed = (int32_t)k;
    if (!finite || !fin(true_rr) || !fin(r_norm)) {
      status = -3;
      break;
    }
    if (r_norm <= tol) {
      status = 0;
      break;
    }
    const float rho_new = dot_f(r, z, n);
    if (!fin(rho_new) || rho_new <= 0.0f) {
      status = -2;
      break;
    }
    const float beta = rho_new / rho;
    if (!fin(beta)) {
      status = -3;
      break;
    }
    for (int64_t i = 0; i < n; ++i) p[i] = z[i] + beta * p[i];
    rho = rho_new;
  }
  *info = status;
  *residual = sqrtf(max0f(true_rr));
  *iterations = completed;
done:
  free(r);
  free(z);
  free(p);
  free(ap);
  return 0;
}

/* ---------------------------------------------------------------------- */
/* BiCGSTAB (src/linalg/bicgstab/bicgstab.cpp:80-362, csr_bicgstab_cpu_impl)
 * and MINRES (src/linalg/minres/minres.cpp:68-312, csr_minres_cpu_impl),
 * float32, the solver SpMV summed from zero.  Dot products are sequential
 * double sums; scalars double; vectors float, each update rounded once. */

static double dot_d(const float *a, const float *b, int64_t n) {
  double acc = 0.0;
  for (int64_t i = 0; i < n; ++i) acc += (double)a[i] * (double)b[i];
  return acc;
}

/* bicgstab.cpp:43-49 */
static int near_zero_dot(double value, double lhs_norm2, double rhs_norm2) {
  const double prod = lhs_norm2 * rhs_norm2;
  const double scale = sqrt(max0(prod));
  const double tol = (double)FLT_EPSILON * (scale > 1.0 ? scale : 1.0);
  return !isfinite(scale) || fabs(value) <= tol;
}

/* dst = b - A x (bicgstab.cpp:130-149): returns float(sqrt(sum dst^2)) and
 * *finite (every dst, A x and x entry, the sum and the norm finite). */
static float bi_true_residual(int it, int64_t n, const float *data, const void *indices,
                              const void *indptr, const float *b, const float *x, float *ax,
                              float *dst, int *finite) {
  cg_spmv(it, n, data, indices, indptr, x, ax);
  double rr = 0.0;
  int ok = 1;
  for (int64_t i = 0; i < n; ++i) {
    const float ri = b[i] - ax[i];
    ok = ok && fin(ri) && fin(ax[i]) && fin(x[i]);
    dst[i] = ri;
    rr += (double)ri * (double)ri;
  }
  const float norm = (float)sqrt(max0(rr));
  *finite = ok && isfinite(rr) && fin(norm);
  return norm;
}

int oracle_csr_bicgstab(int it, int64_t n, const float *data, const void *indices,
                        const void *indptr, const float *b, const float *x0, float *x, float rtol,
                        float atol, int64_t maxiter, int32_t *info, float *residual,
                        int32_t *iterations) {
  const size_t bytes = (size_t)(n > 0 ? n : 1) * sizeof(float);
  float *r = (float *)malloc(bytes), *r_hat = (float *)malloc(bytes), *p = (float *)malloc(bytes);
  float *v = (float *)malloc(bytes), *s = (float *)malloc(bytes), *t = (float *)malloc(bytes);
  float *ax = (float *)malloc(bytes);
  int32_t status = 0, completed = 0;
  float residual_norm = 0.0f;
  if (!r || !r_hat || !p || !v || !s || !t || !ax) {
    free(r); free(r_hat); free(p); free(v); free(s); free(t); free(ax);
    return -1;
  }
  memset(p, 0, bytes);
  memset(v, 0, bytes);
  memcpy(x, x0, (size_t)n * sizeof(float));
  double b_norm2 = 0.0;
  int setup_finite = 1;
  for (int64_t i = 0; i < n; ++i) {
    b_norm2 += (double)b[i] * (double)b[i];
    setup_finite = setup_finite && fin(b[i]) && fin(x[i]);
  }
  const float b_norm = (float)sqrt(max0(b_norm2));
  const float scaled = rtol * b_norm;
  const float tol = atol > scaled ? atol : scaled;
  int finite = 1;
  residual_norm = bi_true_residual(it, n, data, indices, indptr, b, x, ax, r, &finite);
  memcpy(r_hat, r, (size_t)n * sizeof(float));
  if (!setup_finite || !fin(b_norm) || !fin(tol) || !finite) {
    status = -3;
    goto done;
  }
  if (residual_norm <= tol) {
    status = 0;
    goto done;
  }
  status = maxiter > 0 ? (int32_t)maxiter : 1;
  double rho_prev = 1.0, alpha = 1.0, omega = 1.0;
  for (int64_t k = 1; k <= maxiter; ++k) {
    const double rho = dot_d(r_hat, r, n);
    const double r_hat_norm2 = dot_d(r_hat, r_hat, n);
    const double r_norm2 = dot_d(r, r, n);
    if (!isfinite(rho) || !isfinite(r_hat_norm2) || !isfinite(r_norm2)) {
      status = -3;
      completed = (int32_t)(k - 1);
      break;
    }
    if (near_zero_dot(rho, r_hat_norm2, r_norm2)) {
      status = -1;
      completed = (int32_t)(k - 1);
      break;
    }
    if (k == 1) {
      memcpy(p, r, (size_t)n * sizeof(float));
    } else {
      if (fabs(omega) <= (double)FLT_EPSILON) {
        status = -1;
        completed = (int32_t)(k - 1);
        break;
      }
      const double beta = (rho / rho_prev) * (alpha / omega);
      if (!isfinite(beta)) {
        status = -3;
        completed = (int32_t)(k - 1);
        break;
      }
      int ok = 1;
      for (int64_t i = 0; i < n; ++i) {
        const double pi = (double)r[i] + beta * ((double)p[i] - omega * (double)v[i]);
        p[i] = (float)pi;
        ok = ok && isfinite(pi) && fin(p[i]);
      }
      if (!ok) {
        status = -3;
        completed = (int32_t)(k - 1);
        break;
      }
    }
    cg_spmv(it, n, data, indices, indptr, p, v);
    const double alpha_den = dot_d(r_hat, v, n);
    const double v_norm2 = dot_d(v, v, n);
    if (!isfinite(alpha_den) || !isfinite(v_norm2)) {
      status = -3;
      completed = (int32_t)(k - 1);
      break;
    }
    if (near_zero_dot(alpha_den, r_hat_norm2, v_norm2)) {
      status = -1;
      completed = (int32_t)(k - 1);
      break;
    }
    alpha = rho / alpha_den;
    if (!isfinite(alpha)) {
      status = -3;
      completed = (int32_t)(k - 1);
      break;
    }
    double s_norm2 = 0.0;
    int ok = 1;
    for (int64_t i = 0; i < n; ++i) {
      const double si = (double)r[i] - alpha * (double)v[i];
      const double xi = (double)x[i] + alpha * (double)p[i];
      s[i] = (float)si;
      x[i] = (float)xi;
      s_norm2 += si * si;
      ok = ok && isfinite(si) && isfinite(xi) && fin(s[i]) && fin(x[i]);
    }
    completed = (int32_t)k;
    const float s_norm = (float)sqrt(max0(s_norm2));
    if (!ok || !isfinite(s_norm2) || !fin(s_norm)) {
      status = -3;
      break;
    }
    if (s_norm <= tol) {
      int tf = 1;
      const float true_norm = bi_true_residual(it, n, data, indices, indptr, b, x, ax, ax, &tf);
      if (!tf) {
        status = -3;
        residual_norm = true_norm;
        break;
      }
      if (true_norm <= tol) {
        status = 0;
        residual_norm = true_norm;
        break;
      }
    }
    cg_spmv(it, n, data, indices, indptr, s, t);
    const double omega_num = dot_d(t, s, n);
    const double omega_den = dot_d(t, t, n);
    if (!isfinite(omega_num) || !isfinite(omega_den)) {
      status = -3;
      break;
    }
    if (near_zero_dot(omega_den, omega_den, 1.0)) {
      status = -1;
      break;
    }
    omega = omega_num / omega_den;
    if (!isfinite(omega)) {
      status = -3;
      break;
    }
    double r_norm2_new = 0.0;
    ok = 1;
    for (int64_t i = 0; i < n; ++i) {
      const double xi = (double)x[i] + omega * (double)s[i];
      const double ri = (double)s[i] - omega * (double)t[i];
      x[i] = (float)xi;
      r[i] = (float)ri;
      r_norm2_new += ri * ri;
      ok = ok && isfinite(xi) && isfinite(ri) && fin(x[i]) && fin(r[i]);
    }
    residual_norm = (float)sqrt(max0(r_norm2_new));
    if (!ok || !isfinite(r_norm2_new) || !fin(residual_norm)) {
      status = -3;
      break;
    }
    if (residual_norm <= tol) {
      int tf = 1;
      const float true_norm = bi_true_residual(it, n, data, indices, indptr, b, x, ax, r, &tf);
      if (!tf) {
        status = -3;
        residual_norm = true_norm;
        break;
      }
      residual_norm = true_norm;
      if (true_norm <= tol) {
        status = 0;
        break;
      }
    }
    if (fabs(omega) <= (double)FLT_EPSILON) {
      status = -1;
      break;
    }
    rho_prev = rho;
  }
  if (status > 0 || status == -1) {
    int tf = 1;
    const float true_norm = bi_true_residual(it, n, data, indices, indptr, b, x, ax, r, &tf);
    residual_norm = true_norm;
    if (!tf) status = -3;
    else if (true_norm <= tol) status = 0;
  }
done:
  *info = status;
  *residual = residual_norm;
  *iterations = completed;
  free(r); free(r_hat); free(p); free(v); free(s); free(t); free(ax);
  return 0;
}

/* ---------------------------------------------------------------------- */
/* BiCGSTAB with a Jacobi preconditioner: the reference's
 * left_preconditioned_bicgstab_host (src/preconditioners/bicgstab/
 * bicgstab.cpp:140-421) with apply(v)[i] = inv_diag[i] * v[i] in float
 * (csr_bicgstab_jacobi_cpu_impl, bicgstab.cpp:425-521).  Against
 * oracle_csr_bicgstab: ||b|| is rounded to float before its square root
 * (norm_float, src/linalg/common/common.h:56-73); x advances along
 * p_hat = M p and s_hat = M s, which the SpMVs take; a failed true-residual
 * evaluation (a non-finite A x entry, residual entry, sum or norm: the
 * reference's exception) ends the solve with status -3 and leaves the
 * reported residual as it was (+inf before the first iteration); the
 * reported residual follows ||s|| after the s update. */

/* true_residual_into (bicgstab.cpp:166-192): 0 where the reference throws. */
static int bj_true_residual(int it, int64_t n, const float *data, const void *indices,
                            const void *indptr, const float *b, const float *x, float *ax,
                            float *dst, float *norm_out) {
  cg_spmv(it, n, data, indices, indptr, x, ax);
  for (int64_t i = 0; i < n; ++i)
    if (!fin(ax[i])) return 0;
  double rr = 0.0;
  int ok = 1;
  for (int64_t i = 0; i < n; ++i) {
    const float ri = b[i] - ax[i];
    dst[i] = ri;
    rr += (double)ri * (double)ri;
    ok = ok && fin(ri);
  }
  const float norm = (float)sqrt(max0(rr));
  if (!ok || !isfinite(rr) || !fin(norm)) return 0;
  *norm_out = norm;
  return 1;
}

/* out = inv_diag * src in float; returns 1 when every entry is finite. */
static int bj_apply(int64_t n, const float *inv_diag, const float *src, float *out) {
  int ok = 1;
  for (int64_t i = 0; i < n; ++i) {
    out[i] = inv_diag[i] * src[i];
    ok = ok && fin(out[i]);
  }
  return ok;
}

static int all_finite(int64_t n, const float *v) {
  for (int64_t i = 0; i < n; ++i)
    if (!fin(v[i])) return 0;
  return 1;
}

int oracle_csr_bicgstab_jacobi(int it, int64_t n, const float *data, const void *indices,
                               const void *indptr, const float *b, const float *x0,
                               const float *inv_diag, float *x, float rtol, float atol,
                               int64_t maxiter, int32_t *info, float *residual,
                               int32_t *iterations) {
  const size_t bytes = (size_t)(n > 0 ? n : 1) * sizeof(float);
  float *buf = (float *)calloc(9, bytes);
  if (!buf) return -1;
  const size_t m = bytes / sizeof(float);
  float *r = buf, *r_hat = buf + m, *p = buf + 2 * m, *p_hat = buf + 3 * m, *v = buf + 4 * m;
  float *s = buf + 5 * m, *s_hat = buf + 6 * m, *t = buf + 7 * m, *ax = buf + 8 * m;
  int32_t status = maxiter > 0 ? (int32_t)maxiter : 1, completed = 0;
  float residual_norm = INFINITY;
  memcpy(x, x0, (size_t)n * sizeof(float));
  double bb = 0.0;
  int setup_finite = 1;
  for (int64_t i = 0; i < n; ++i) {
    bb += (double)b[i] * (double)b[i];
    setup_finite = setup_finite && fin(b[i]) && fin(x[i]);
  }
  const float b_norm = sqrtf(max0f((float)bb));
  const float scaled = rtol * b_norm;
  const float tol = atol > scaled ? atol : scaled;
  if (!setup_finite || !fin(b_norm) || !fin(tol)) {
    status = -3;
    goto done;
  }
  if (!bj_true_residual(it, n, data, indices, indptr, b, x, ax, r, &residual_norm)) {
    status = -3;
    goto done;
  }
  memcpy(r_hat, r, (size_t)n * sizeof(float));
  if (residual_norm <= tol) {
    status = 0;
    goto done;
  }
  double rho_prev = 1.0, alpha = 1.0, omega = 1.0;
  for (int64_t k = 1; k <= maxiter; ++k) {
    const double rho = dot_d(r_hat, r, n);
    const double r_hat_norm2 = dot_d(r_hat, r_hat, n);
    const double r_norm2 = dot_d(r, r, n);
    if (!isfinite(rho) || !isfinite(r_hat_norm2) || !isfinite(r_norm2)) {
      status = -3;
      completed = (int32_t)(k - 1);
      break;
    }
    if (near_zero_dot(rho, r_hat_norm2, r_norm2)) {
      status = -1;
      completed = (int32_t)(k - 1);
      break;
    }
    if (k == 1) {
      memcpy(p, r, (size_t)n * sizeof(float));
    } else {
      if (fabs(omega) <= (double)FLT_EPSILON) {
        status = -1;
        completed = (int32_t)(k - 1);
        break;
      }
      const double beta = (rho / rho_prev) * (alpha / omega);
      if (!isfinite(beta)) {
        status = -3;
        completed = (int32_t)(k - 1);
        break;
      }
      int ok = 1;
      for (int64_t i = 0; i < n; ++i) {
        const double pi = (double)r[i] + beta * ((double)p[i] - omega * (double)v[i]);
        p[i] = (float)pi;
        ok = ok && isfinite(pi) && fin(p[i]);
      }
      if (!ok) {
        status = -3;
        completed = (int32_t)(k - 1);
        break;
      }
    }
    if (!bj_apply(n, inv_diag, p, p_hat)) {
      status = -3;
      completed = (int32_t)(k - 1);
      break;
    }
    cg_spmv(it, n, data, indices, indptr, p_hat, v);
    if (!all_finite(n, v)) {
      status = -3;
      completed = (int32_t)(k - 1);
      break;
    }
    const double alpha_den = dot_d(r_hat, v, n);
    const double v_norm2 = dot_d(v, v, n);
    if (!isfinite(alpha_den) || !isfinite(v_norm2)) {
      status = -3;
      completed = (int32_t)(k - 1);
      break;
    }
    if (near_zero_dot(alpha_den, r_hat_norm2, v_norm2)) {
      status = -1;
      completed = (int32_t)(k - 1);
      break;
    }
    alpha = rho / alpha_den;
    if (!isfinite(alpha)) {
      status = -3;
      completed = (int32_t)(k - 1);
      break;
    }
    double s_norm2 = 0.0;
    int ok = 1;
    for (int64_t i = 0; i < n; ++i) {
      const double si = (double)r[i] - alpha * (double)v[i];
      const double xi = (double)x[i] + alpha * (double)p_hat[i];
      s[i] = (float)si;
      x[i] = (float)xi;
      s_norm2 += si * si;
      ok = ok && isfinite(si) && isfinite(xi) && fin(s[i]) && fin(x[i]);
    }
    completed = (int32_t)k;
    residual_norm = (float)sqrt(max0(s_norm2));
    if (!ok || !isfinite(s_norm2) || !fin(residual_norm)) {
      status = -3;
      break;
    }
    if (residual_norm <= tol) {
      float true_norm = 0.0f;
      if (!bj_true_residual(it, n, data, indices, indptr, b, x, ax, t, &true_norm)) {
        status = -3;
        break;
      }
      if (true_norm <= tol) {
        status = 0;
        residual_norm = true_norm;
        break;
      }
    }
    if (!bj_apply(n, inv_diag, s, s_hat)) {
      status = -3;
      break;
    }
    cg_spmv(it, n, data, indices, indptr, s_hat, t);
    if (!all_finite(n, t)) {
      status = -3;
      break;
    }
    const double omega_num = dot_d(t, s, n);
    const double omega_den = dot_d(t, t, n);
    if (!isfinite(omega_num) || !isfinite(omega_den)) {
      status = -3;
      break;
    }
    if (near_zero_dot(omega_den, omega_den, 1.0)) {
      status = -1;
      break;
    }
    omega = omega_num / omega_den;
    if (!isfinite(omega)) {
      status = -3;
      break;
    }
    double r_norm2_new = 0.0;
    ok = 1;
    for (int64_t i = 0; i < n; ++i) {
      const double xi = (double)x[i] + omega * (double)s_hat[i];
      const double ri = (double)s[i] - omega * (double)t[i];
      x[i] = (float)xi;
      r[i] = (float)ri;
      r_norm2_new += ri * ri;
      ok = ok && isfinite(xi) && isfinite(ri) && fin(x[i]) && fin(r[i]);
    }
    residual_norm = (float)sqrt(max0(r_norm2_new));
    if (!ok || !isfinite(r_norm2_new) || !fin(residual_norm)) {
      status = -3;
      break;
    }
    if (residual_norm <= tol) {
      float true_norm = 0.0f;
      if (!bj_true_residual(it, n, data, indices, indptr, b, x, ax, r, &true_norm)) {
        status = -3;
        break;
      }
      residual_norm = true_norm;
      if (true_norm <= tol) {
        status = 0;
        break;
      }
    }
    if (fabs(omega) <= (double)FLT_EPSILON) {
      status = -1;
      break;
    }
    rho_prev = rho;
  }
  if (status > 0 || status == -1) {
    float true_norm = 0.0f;
    if (!bj_true_residual(it, n, data, indices, indptr, b, x, ax, r, &true_norm)) {
      status = -3;
    } else {
      residual_norm = true_norm;
      if (true_norm <= tol) status = 0;
    }
  }
done:
  *info = status;
  *residual = residual_norm;
  *iterations = completed;
  free(buf);
  return 0;
}

/* (A - shift I) x residual (minres.cpp:68-91): work = A x, then
 * ai = work - shift x, ri = b - ai in float; *finite: every ai, ri and the
 * norm finite. */
static float mr_true_residual(int it, int64_t n, const float *data, const void *indices,
                              const void *indptr, const float *b, const float *x, float *work,
                              float shift, int *finite) {
  cg_spmv(it, n, data, indices, indptr, x, work);
  double rr = 0.0;
  int ok = 1;
  for (int64_t i = 0; i < n; ++i) {
    const float ai = work[i] - shift * x[i];
    const float ri = b[i] - ai;
    rr += (double)ri * (double)ri;
    ok = ok && fin(ai) && fin(ri);
  }
  const float norm = (float)sqrt(max0(rr));
  *finite = ok && fin(norm);
  return norm;
}

/* MINRES, plain (inv_diag NULL) or with the Jacobi preconditioner
 * M = diag(inv_diag) (src/preconditioners/minres/minres.cpp:93-330,
 * csr_minres_jacobi_cpu_impl): there y = M r2 in float instead of y = r2;
 * an inverse diagonal entry that is not > 0 stops the start with -2 (after
 * the non-finite test, before the convergence test); and the non-positive
 * or non-finite beta tests give -2 instead of -1. */
static int minres_loop(int it, int64_t n, const float *data, const void *indices,
                       const void *indptr, const float *b, const float *x0, const float *inv_diag,
                       float *x, float rtol, float atol, int64_t maxiter, float shift,
                       int32_t *info, float *residual, int32_t *iterations) {
  const int32_t beta_fail = inv_diag ? -2 : -1;
  const size_t bytes = (size_t)(n > 0 ? n : 1) * sizeof(float);
  float *r1 = (float *)calloc(1, bytes), *r2 = (float *)calloc(1, bytes);
  float *y = (float *)calloc(1, bytes), *v = (float *)calloc(1, bytes);
  float *w = (float *)calloc(1, bytes), *w2 = (float *)calloc(1, bytes);
  float *av = (float *)calloc(1, bytes);
  if (!r1 || !r2 || !y || !v || !w || !w2 || !av) {
    free(r1); free(r2); free(y); free(v); free(w); free(w2); free(av);
    return -1;
  }
  memcpy(x, x0, (size_t)n * sizeof(float));
  double b_norm2 = 0.0;
  for (int64_t i = 0; i < n; ++i) b_norm2 += (double)b[i] * (double)b[i];
  const float b_norm = (float)sqrt(max0(b_norm2));
  const float scaled = rtol * b_norm;
  const float tol = atol > scaled ? atol : scaled;
  int32_t status = maxiter > 0 ? (int32_t)maxiter : 1;
  int32_t completed = 0;
  /* the finite flag of minres.cpp:161-165 is reset by the residual helper */
  int finite = 1;
  float true_residual = mr_true_residual(it, n, data, indices, indptr, b, x, av, shift, &finite);
  if (!finite) {
    status = -3;
    goto done;
  }
  if (inv_diag) {
    for (int64_t i = 0; i < n; ++i) {
      if (!(inv_diag[i] > 0.0f)) {
        status = -2;
        goto done;
      }
    }
  }
  if (true_residual <= tol) {
    status = 0;
    goto done;
  }
  if (maxiter == 0) goto done;
  for (int64_t i = 0; i < n; ++i) {
    const float ai = av[i] - shift * x[i];
    const float ri = b[i] - ai;
    r2[i] = ri;
    y[i] = inv_diag ? inv_diag[i] * ri : ri;
  }
  double beta_inner = (double)(float)dot_d(r2, y, n);
  if (!isfinite(beta_inner) || beta_inner <= 0.0) {
    status = beta_fail;
    goto done;
  }
  const double eps = (double)FLT_EPSILON;
  double beta = sqrt(beta_inner), oldb = 0.0, dbar = 0.0, epsln = 0.0, phibar = beta;
  double cs = -1.0, sn = 0.0;
  for (int64_t k = 1; k <= maxiter; ++k) {
    if (!isfinite(beta) || beta <= eps) {
      status = beta_fail;
      break;
    }
    const double inv_beta = 1.0 / beta;
    for (int64_t i = 0; i < n; ++i) v[i] = (float)(inv_beta * (double)y[i]);
    cg_spmv(it, n, data, indices, indptr, v, av);
    for (int64_t i = 0; i < n; ++i) av[i] = av[i] - shift * v[i];
    if (k >= 2) {
      if (!isfinite(oldb) || fabs(oldb) <= eps) {
        status = -1;
        break;
      }
      const float prev_scale = (float)(beta / oldb);
      for (int64_t i = 0; i < n; ++i) av[i] = av[i] - prev_scale * r1[i];
    }
    const double alfa = (double)(float)dot_d(v, av, n);
    if (!isfinite(alfa)) {
      status = -3;
      break;
    }
    const float diag_scale = (float)(alfa / beta);
    for (int64_t i = 0; i < n; ++i) av[i] = av[i] - diag_scale * r2[i];
    /* r1 <- r2, r2 <- av, y = M r2 (the old r1 becomes scratch) */
    float *old_r1 = r1;
    r1 = r2;
    r2 = av;
    av = old_r1;
    for (int64_t i = 0; i < n; ++i) y[i] = inv_diag ? inv_diag[i] * r2[i] : r2[i];
    oldb = beta;
    beta_inner = (double)(float)dot_d(r2, y, n);
    if (!isfinite(beta_inner) || beta_inner < 0.0) {
      status = beta_fail;
      break;
    }
    beta = sqrt(max0(beta_inner));
    const double oldeps = epsln;
    const double delta = cs * dbar + sn * alfa;
    const double gbar = sn * dbar - cs * alfa;
    epsln = sn * beta;
    dbar = -cs * beta;
    double gamma = hypot(gbar, beta);
    if (!isfinite(gamma)) {
      status = -3;
      break;
    }
    gamma = gamma > eps ? gamma : eps;
    cs = gbar / gamma;
    sn = beta / gamma;
    const double phi = cs * phibar;
    phibar = sn * phibar;
    if (!isfinite(phi) || !isfinite(phibar)) {
      status = -3;
      break;
    }
    int ok = 1;
    for (int64_t i = 0; i < n; ++i) {
      const float prev_w1 = w2[i];
      const float prev_w2 = w[i];
      w2[i] = prev_w2;
      w[i] = (float)(((double)v[i] - oldeps * (double)prev_w1 - delta * (double)prev_w2) / gamma);
      x[i] = x[i] + (float)(phi * (double)w[i]);
      ok = ok && fin(w[i]) && fin(x[i]);
    }
    completed = (int32_t)k;
    if (!ok) {
      status = -3;
      break;
    }
    true_residual = mr_true_residual(it, n, data, indices, indptr, b, x, av, shift, &finite);
    if (!finite) {
      status = -3;
      break;
    }
    if (true_residual <= tol) {
      status = 0;
      break;
    }
    if (beta <= eps) {
      status = -1;
      break;
    }
  }
done:
  *info = status;
  *residual = true_residual;
  *iterations = completed;
  free(r1); free(r2); free(y); free(v); free(w); free(w2); free(av);
  return 0;
}

int oracle_csr_minres(int it, int64_t n, const float *data, const void *indices,
                      const void *indptr, const float *b, const float *x0, float *x, float rtol,
                      float atol, int64_t maxiter, float shift, int32_t *info, float *residual,
                      int32_t *iterations) {
  return minres_loop(it, n, data, indices, indptr, b, x0, NULL, x, rtol, atol, maxiter, shift,
                     info, residual, iterations);
}

int oracle_csr_minres_jacobi(int it, int64_t n, const float *data, const void *indices,
                             const void *indptr, const float *b, const float *x0,
                             const float *inv_diag, float *x, float rtol, float atol,
                             int64_t maxiter, float shift, int32_t *info, float *residual,
                             int32_t *iterations) {
  return minres_loop(it, n, data, indices, indptr, b, x0, inv_diag, x, rtol, atol, maxiter, shift,
                     info, residual, iterations);
}

/* ---------------------------------------------------------------------- */
/* Restarted GMRES (src/linalg/gmres/gmres.cpp:58-220, csr_gmres_impl) over
 * the CPU Arnoldi factorisation (src/linalg/arnoldi/arnoldi.cpp:79-159,
 * csr_arnoldi_cpu_impl) and the small upper-Hessenberg least-squares solve
 * by Givens QR (src/linalg/common/common.h:143-234,
 * least_squares_upper_hessenberg_givens_qr), float32 values; the solver SpMV
 * is csr_spmv_float (common.h:35-45), summed from zero. */

/* norm_float (common.h:56-73): float(sqrt(max(float(sum of double
 * squares), 0))). */
static float norm_f(const float *v, int64_t n) {
  const float dd = dot_f(v, v, n);
  return sqrtf(max0f(dd));
}

/* k Arnoldi steps from v0: h is (k+1) x k row-major, basis n x (k+1)
 * row-major (basis[row * (k+1) + col]); *used = steps taken.  Two passes of
 * modified Gram-Schmidt per step, each coefficient a double sum of float
 * products, subtracted in float; the step ends early when the new norm is
 * at most FLT_EPSILON. */
/* With inv_diag (the Jacobi Arnoldi, src/preconditioners/gmres/gmres.cpp:
 * 342-447): the basis of M A, M = diag(inv_diag) - w = M (A q) in float -
 * no step when v0 or inv_diag holds a non-finite entry, and a non-finite
 * new norm ends the factorisation with zero steps. */
static int arnoldi_impl(int it, int64_t n, const float *data, const void *indices,
                        const void *indptr, const float *inv_diag, const float *v0, int64_t k,
                        float *h, float *basis, int32_t *used_out) {
  const int64_t cols = k + 1;
  float *w = (float *)malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
  float *q = (float *)malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
  if (!w || !q) {
    free(w);
    free(q);
    return -1;
  }
  memset(h, 0, (size_t)cols * (size_t)k * sizeof(float));
  memset(basis, 0, (size_t)n * (size_t)cols * sizeof(float));
  double v_norm2 = 0.0;
  int inputs_ok = 1;
  for (int64_t i = 0; i < n; ++i) {
    v_norm2 += (double)v0[i] * (double)v0[i];
    if (inv_diag) inputs_ok = inputs_ok && fin(v0[i]) && fin(inv_diag[i]);
  }
  const float v_norm = (float)sqrt(v_norm2 < 0.0 ? 0.0 : v_norm2);
  const float eps = FLT_EPSILON;
  if (inv_diag && (!inputs_ok || !fin(v_norm))) {
    *used_out = 0;
    free(w);
    free(q);
    return 0;
  }
  for (int64_t i = 0; i < n; ++i)
    basis[i * cols] = v_norm <= eps ? (i == 0 ? 1.0f : 0.0f) : v0[i] / v_norm;
  int32_t used = 0;
  for (int64_t j = 0; j < k; ++j) {
    for (int64_t i = 0; i < n; ++i) q[i] = basis[i * cols + j];
    cg_spmv(it, n, data, indices, indptr, q, w);
    if (inv_diag)
      for (int64_t row = 0; row < n; ++row) w[row] = w[row] * inv_diag[row];
    for (int pass = 0; pass < 2; ++pass) {
      for (int64_t col = 0; col <= j; ++col) {
        double coeff = 0.0;
        for (int64_t row = 0; row < n; ++row) {
          const float prod = basis[row * cols + col] * w[row];
          coeff += (double)prod;
        }
        const float c = (float)coeff;
        h[col * k + j] = h[col * k + j] + c;
        for (int64_t row = 0; row < n; ++row) {
          const float t = c * basis[row * cols + col];
          w[row] = w[row] - t;
        }
      }
    }
    const float h_next = norm_f(w, n);
    h[(j + 1) * k + j] = h_next;
    used = (int32_t)(j + 1);
    if (inv_diag && !fin(h_next)) {
      used = 0;
      break;
    }
    if (h_next <= eps) break;
    for (int64_t row = 0; row < n; ++row) basis[row * cols + j + 1] = w[row] / h_next;
  }
  *used_out = used;
  free(w);
  free(q);
  return 0;
}

int oracle_csr_arnoldi(int it, int64_t n, const float *data, const void *indices,
                       const void *indptr, const float *v0, int64_t k, float *h, float *basis,
                       int32_t *used_out) {
  return arnoldi_impl(it, n, data, indices, indptr, NULL, v0, k, h, basis, used_out);
}

int oracle_csr_arnoldi_jacobi(int it, int64_t n, const float *data, const void *indices,
                              const void *indptr, const float *inv_diag, const float *v0,
                              int64_t k, float *h, float *basis, int32_t *used_out) {
  return arnoldi_impl(it, n, data, indices, indptr, inv_diag, v0, k, h, basis, used_out);
}

/* min ||a y - b|| for an upper-Hessenberg a of rows = cols + 1 (row-major,
 * double) by Givens rotations; returns 0, or 1 where the reference throws
 * (non-finite input, rank-deficient matrix, degenerate rotation or R
 * factor, non-finite solution). */
static int lsq_hessenberg(const double *a, const double *b, int64_t rows, int64_t cols, double *y) {
  if (rows != cols + 1 || rows <= 1 || cols <= 0) return 1;
  double *r = (double *)malloc((size_t)(rows * cols) * sizeof(double));
  double *rhs = (double *)malloc((size_t)rows * sizeof(double));
  int err = 0;
  if (!r || !rhs) {
    free(r);
    free(rhs);
    return 1;
  }
  memcpy(r, a, (size_t)(rows * cols) * sizeof(double));
  memcpy(rhs, b, (size_t)rows * sizeof(double));
  double scale = 0.0;
  for (int64_t i = 0; i < rows * cols; ++i) {
    if (!isfinite(r[i])) err = 1;
    const double m = fabs(r[i]);
    if (m > scale) scale = m;
  }
  for (int64_t i = 0; i < rows; ++i)
    if (!isfinite(rhs[i])) err = 1;
  const double big = (double)(rows > cols ? rows : cols);
  const double rank_tol = DBL_EPSILON * big * (scale > 1.0 ? scale : 1.0);
  if (!err && scale <= rank_tol) err = 1;
  for (int64_t col = 0; !err && col < cols; ++col) {
    const int64_t row = col + 1;
    const double pivot = r[col * cols + col];
    const double entry = r[row * cols + col];
    if (entry == 0.0) continue;
    const double radius = hypot(pivot, entry);
    if (!isfinite(radius) || radius <= rank_tol) {
      err = 1;
      break;
    }
    const double c = pivot / radius;
    const double s = entry / radius;
    for (int64_t j = col; j < cols; ++j) {
      const double top = r[col * cols + j];
      const double bottom = r[row * cols + j];
      r[col * cols + j] = c * top + s * bottom;
      r[row * cols + j] = -s * top + c * bottom;
    }
    const double rt = rhs[col], rb = rhs[row];
    rhs[col] = c * rt + s * rb;
    rhs[row] = -s * rt + c * rb;
  }
  for (int64_t row = cols - 1; !err && row >= 0; --row) {
    double sum = rhs[row];
    for (int64_t col = row + 1; col < cols; ++col) sum -= r[row * cols + col] * y[col];
    const double diag = r[row * cols + row];
    if (!isfinite(diag) || fabs(diag) <= rank_tol) {
      err = 1;
      break;
    }
    y[row] = sum / diag;
    if (!isfinite(y[row])) err = 1;
  }
  free(r);
  free(rhs);
  return err;
}

/* b - A x into r; returns norm_float(r), *finite = every r entry and the
 * norm finite. */
static float gm_residual(int it, int64_t n, const float *data, const void *indices,
                         const void *indptr, const float *b, const float *x, float *ax, float *r,
                         int *finite) {
  cg_spmv(it, n, data, indices, indptr, x, ax);
  int ok = 1;
  for (int64_t i = 0; i < n; ++i) {
    r[i] = b[i] - ax[i];
    ok = ok && fin(r[i]);
  }
  const float nr = norm_f(r, n);
  *finite = ok && fin(nr);
  return nr;
}

/* Restarted GMRES: info 0 converged, maxiter (1 when maxiter is 0) when the
 * budget ran out, -1 a failed least-squares solve, -3 non-finite; residual
 * the last true residual norm (infinity when the inputs are not finite);
 * iterations the Arnoldi steps taken. */
/* With inv_diag: GMRES with the Jacobi preconditioner
 * (src/preconditioners/gmres/gmres.cpp:572-748, csr_gmres_jacobi_impl):
 * each cycle starts from z0 = M r (its norm ||M r|| is the least-squares
 * right-hand side, at most FLT_EPSILON: -1) over the Jacobi Arnoldi basis;
 * the true residual ||r|| decides convergence; a non-finite inverse
 * diagonal entry is a non-finite input; the least-squares solution is not
 * tested on its own (a non-finite update row is). */
static int gmres_impl(int it, int64_t n, const float *data, const void *indices,
                      const void *indptr, const float *b, const float *x0, const float *inv_diag,
                      float *x, float rtol, float atol, int64_t restart, int64_t maxiter,
                      int32_t *info, float *residual, int32_t *iterations) {
  const size_t nb = (size_t)(n > 0 ? n : 1) * sizeof(float);
  const int64_t kmax = restart < maxiter ? restart : maxiter;
  const int64_t kcap = (kmax < n ? kmax : n) > 0 ? (kmax < n ? kmax : n) : 1;
  float *r = (float *)malloc(nb), *ax = (float *)malloc(nb), *v0 = (float *)malloc(nb);
  float *z0 = (float *)malloc(nb);
  float *h = (float *)malloc((size_t)((kcap + 1) * kcap) * sizeof(float));
  float *basis = (float *)malloc((size_t)n * (size_t)(kcap + 1) * sizeof(float));
  double *hd = (double *)malloc((size_t)((kcap + 1) * kcap) * sizeof(double));
  double *e1 = (double *)malloc((size_t)(kcap + 1) * sizeof(double));
  double *y = (double *)malloc((size_t)kcap * sizeof(double));
  if (!r || !ax || !v0 || !z0 || !h || !basis || !hd || !e1 || !y) {
    free(r); free(ax); free(v0); free(z0); free(h); free(basis); free(hd); free(e1); free(y);
    return -1;
  }
  memcpy(x, x0, (size_t)n * sizeof(float));
  const float b_norm = norm_f(b, n);
  const float scaled = rtol * b_norm;
  const float tol = atol > scaled ? atol : scaled;
  int64_t iters = 0;
  int32_t status = maxiter > 0 ? (int32_t)maxiter : 1;
  float res = INFINITY;
  int inputs_ok = fin(b_norm) && fin(tol);
  for (int64_t i = 0; i < n; ++i)
    inputs_ok = inputs_ok && fin(x[i]) && fin(b[i]) && (!inv_diag || fin(inv_diag[i]));
  if (!inputs_ok) {
    status = -3;
    goto done;
  }
  while (iters < maxiter) {
    int finite = 1;
    float beta = gm_residual(it, n, data, indices, indptr, b, x, ax, r, &finite);
    res = beta;
    if (inv_diag) {
      for (int64_t i = 0; i < n; ++i) {
        z0[i] = inv_diag[i] * r[i];
        finite = finite && fin(z0[i]);
      }
    }
    if (!finite) {
      status = -3;
      break;
    }
    if (res <= tol) {
      status = 0;
      break;
    }
    if (inv_diag) {
      beta = norm_f(z0, n);
      if (!fin(beta) || beta <= FLT_EPSILON) {
        status = -1;
        break;
      }
    }
    int64_t steps = restart;
    if (maxiter - iters < steps) steps = maxiter - iters;
    if (n < steps) steps = n;
    for (int64_t i = 0; i < n; ++i) v0[i] = (inv_diag ? z0[i] : r[i]) / beta;
    int32_t used = 0;
    if (arnoldi_impl(it, n, data, indices, indptr, inv_diag, v0, steps, h, basis, &used) != 0) {
      free(r); free(ax); free(v0); free(z0); free(h); free(basis); free(hd); free(e1); free(y);
      return -1;
    }
    if (used == 0) {
      status = -1;
      break;
    }
    int bad = 0;
    for (int64_t row = 0; row < used + 1; ++row)
      for (int64_t col = 0; col < used; ++col) {
        hd[row * used + col] = (double)h[row * steps + col];
        if (!isfinite(hd[row * used + col])) bad = 1;
      }
    if (bad) {
      status = -3;
      break;
    }
    e1[0] = (double)beta;
    for (int64_t i = 1; i < used + 1; ++i) e1[i] = 0.0;
    if (lsq_hessenberg(hd, e1, used + 1, used, y) != 0) {
      status = -1;
      break;
    }
    for (int64_t c = 0; c < used && !inv_diag; ++c)
      if (!isfinite(y[c])) bad = 1;
    if (bad) {
      status = -3;
      break;
    }
    for (int64_t row = 0; row < n; ++row) {
      double update = 0.0;
      for (int64_t col = 0; col < used; ++col)
        update += (double)basis[row * (steps + 1) + col] * y[col];
      if (!isfinite(update)) {
        bad = 1;
        break;
      }
      x[row] = x[row] + (float)update;
      if (!fin(x[row])) {
        bad = 1;
        break;
      }
    }
    if (bad) {
      status = -3;
      break;
    }
    iters += used;
    if (iters >= maxiter) {
      res = gm_residual(it, n, data, indices, indptr, b, x, ax, r, &finite);
      if (!finite) status = -3;
      else if (res <= tol) status = 0;
      break;
    }
  }
  if (maxiter == 0 && status > 0) {
    int finite = 1;
    res = gm_residual(it, n, data, indices, indptr, b, x, ax, r, &finite);
    if (!finite) status = -3;
    else if (res <= tol) status = 0;
  }
done:
  *info = status;
  *residual = res;
  *iterations = (int32_t)iters;
  free(r); free(ax); free(v0); free(z0); free(h); free(basis); free(hd); free(e1); free(y);
  return 0;
}

int oracle_csr_gmres(int it, int64_t n, const float *data, const void *indices, const void *indptr,
                     const float *b, const float *x0, float *x, float rtol, float atol,
                     int64_t restart, int64_t maxiter, int32_t *info, float *residual,
                     int32_t *iterations) {
  return gmres_impl(it, n, data, indices, indptr, b, x0, NULL, x, rtol, atol, restart, maxiter,
                    info, residual, iterations);
}

int oracle_csr_gmres_jacobi(int it, int64_t n, const float *data, const void *indices,
                            const void *indptr, const float *b, const float *x0,
                            const float *inv_diag, float *x, float rtol, float atol,
                            int64_t restart, int64_t maxiter, int32_t *info, float *residual,
                            int32_t *iterations) {
  return gmres_impl(it, n, data, indices, indptr, b, x0, inv_diag, x, rtol, atol, restart,
                    maxiter, info, residual, iterations);
}

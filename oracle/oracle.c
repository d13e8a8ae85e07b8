/*
 * CPU oracle for the contraction / permutation hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only as the checker (or the timed CPU
 * baseline), never as the thing measured or shipped. The product path
 * (liblinalg_hip.so) has no CPU fallback and never calls into this file.
 *
 * The reference's CPU oracle (crates/cpu, Rust) cannot be compiled here (no Rust toolchain),
 * so this is a C restatement of the reference algorithms, each function citing what it
 * follows. Build: gcc -O2 -ffp-contract=off (no FMA contraction, no reassociation), so every
 * `a * b + c` below rounds twice, exactly as the reference evaluates it.
 *
 * Pinning (tests/test_oracle.py): the gemm functions against the known-answer vectors of
 * crates/cpu/src/invariants.rs:137-243 (tests/golden/cpu_gemm_kats.json), closed forms
 * (identity / permutation / integer matrices), and each other bit for bit; the gather
 * against numpy.transpose on raw words and the complex word table of
 * tests/permutation_test.rs:464-492; the f64 reference against numpy float64 einsum and
 * exact integer cases; the training ops against the reference's own known answers and f64
 * bounds (crates/cpu/src/training.rs, crates/cpu/src/invariants.rs:446-500), the constants'
 * asserted bit patterns, and the exhaustive bf16 table (tests/test_training_oracle.py).
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/*
 * CpuBackend::gemm's accumulation (crates/cpu/src/lib.rs:664-691) over a 2-D strided
 * indexer (crates/cpu/src/lib.rs:651-656): for every (row, col) in row-major order,
 *   acc = (beta == 0) ? +0 : beta * C[row, col]
 *   if (alpha != 0) for inner in 0..k: acc += (alpha * A[row, inner]) * B[inner, col]
 *   C[row, col] = acc
 * Pointers are the views' element-offset bases; strides are in elements. The literal,
 * single-threaded form: what crates/cpu runs.
 */
void oracle_gemm_seq_f32(uint64_t m, uint64_t n, uint64_t k, float alpha, float beta,
                         const float* a, int64_t a_rs, int64_t a_cs,
                         const float* b, int64_t b_rs, int64_t b_cs,
                         float* c, int64_t c_rs, int64_t c_cs) {
    for (uint64_t row = 0; row < m; ++row) {
        for (uint64_t col = 0; col < n; ++col) {
            float* out = c + (int64_t)row * c_rs + (int64_t)col * c_cs;
            float acc = (beta == 0.0f) ? 0.0f : beta * *out;
            if (alpha != 0.0f) {
                for (uint64_t inner = 0; inner < k; ++inner) {
                    const float t = alpha * a[(int64_t)row * a_rs + (int64_t)inner * a_cs];
                    const float p = t * b[(int64_t)inner * b_rs + (int64_t)col * b_cs];
                    acc = acc + p;
                }
            }
            *out = acc;
        }
    }
}

/*
 * The same arithmetic with the loops interchanged (inner outside, columns inside) so it
 * vectorizes across columns and runs rows on several threads. Every output element still
 * sees exactly the operations of oracle_gemm_seq_f32 in the same order -- (alpha*a) rounds,
 * times b rounds, plus acc rounds, k ascending -- so the two are bit-identical (checked by
 * the tests). B is first copied to a dense row-major K x N block (an exact copy) so the
 * column loop is unit stride whatever B's layout.
 *
 * rows: optional list of `nrows` row indices to compute (NULL = all m rows, nrows ignored).
 */
typedef struct {
    uint64_t n, k;
    float alpha, beta;
    const float* a;
    int64_t a_rs, a_cs;
    const float* bd; /* dense K x N */
    float* c;
    int64_t c_rs, c_cs;
    const uint64_t* rows;
    uint64_t first, last; /* range of the row list handled by this worker */
} fast_job;

#define COLS 512

static void* fast_worker(void* arg) {
    const fast_job* j = (const fast_job*)arg;
    float acc[COLS];
    for (uint64_t r = j->first; r < j->last; ++r) {
        const uint64_t row = j->rows ? j->rows[r] : r;
        for (uint64_t c0 = 0; c0 < j->n; c0 += COLS) {
            const uint64_t cn = (j->n - c0 < COLS) ? j->n - c0 : COLS;
            for (uint64_t col = 0; col < cn; ++col) {
                const float cv = j->c[(int64_t)row * j->c_rs + (int64_t)(c0 + col) * j->c_cs];
                acc[col] = (j->beta == 0.0f) ? 0.0f : j->beta * cv;
            }
            if (j->alpha != 0.0f) {
                for (uint64_t inner = 0; inner < j->k; ++inner) {
                    const float t = j->alpha * j->a[(int64_t)row * j->a_rs + (int64_t)inner * j->a_cs];
                    const float* brow = j->bd + inner * j->n + c0;
                    for (uint64_t col = 0; col < cn; ++col) {
                        const float p = t * brow[col];
                        acc[col] = acc[col] + p;
                    }
                }
            }
            for (uint64_t col = 0; col < cn; ++col) {
                j->c[(int64_t)row * j->c_rs + (int64_t)(c0 + col) * j->c_cs] = acc[col];
            }
        }
    }
    return NULL;
}

int oracle_gemm_fast_f32(uint64_t m, uint64_t n, uint64_t k, float alpha, float beta,
                         const float* a, int64_t a_rs, int64_t a_cs,
                         const float* b, int64_t b_rs, int64_t b_cs,
                         float* c, int64_t c_rs, int64_t c_cs,
                         const uint64_t* rows, uint64_t nrows, int threads) {
    const uint64_t count = rows ? nrows : m;
    if (count == 0 || n == 0) return 0;
    float* bd = NULL;
    if (alpha != 0.0f && k > 0) {
        bd = (float*)malloc(sizeof(float) * k * n);
        if (!bd) return -1;
        for (uint64_t i = 0; i < k; ++i)
            for (uint64_t col = 0; col < n; ++col)
                bd[i * n + col] = b[(int64_t)i * b_rs + (int64_t)col * b_cs];
    }
    if (threads < 1) threads = 1;
    if ((uint64_t)threads > count) threads = (int)count;
    fast_job jobs[256];
    pthread_t tids[256];
    if (threads > 256) threads = 256;
    for (int t = 0; t < threads; ++t) {
        fast_job* j = &jobs[t];
        j->n = n;
        j->k = (bd ? k : 0);
        j->alpha = (bd ? alpha : 0.0f);
        j->beta = beta;
        j->a = a;
        j->a_rs = a_rs;
        j->a_cs = a_cs;
        j->bd = bd;
        j->c = c;
        j->c_rs = c_rs;
        j->c_cs = c_cs;
        j->rows = rows;
        j->first = count * (uint64_t)t / (uint64_t)threads;
        j->last = count * (uint64_t)(t + 1) / (uint64_t)threads;
    }
    int rc = 0;
    for (int t = 1; t < threads; ++t) {
        if (pthread_create(&tids[t], NULL, fast_worker, &jobs[t]) != 0) rc = -2;
    }
    fast_worker(&jobs[0]);
    for (int t = 1; t < threads; ++t) pthread_join(tids[t], NULL);
    free(bd);
    return rc;
}

/*
 * gather_words (tests/permutation_test.rs:84-116): the raw 32-bit words of a view in
 * row-major logical order; with `conj` on a complex (two-word) element the second word's
 * sign bit is flipped. `base` is the allocation as words; offset/strides in elements of
 * `w` words. gather_range writes logical elements [first, last) to out[first*w ...): an
 * odometer over the view's indices started at `first`'s mixed-radix decomposition.
 */
static void gather_range(const uint32_t* base, uint32_t w, uint64_t offset, uint32_t rank,
                         const uint64_t* shape, const uint64_t* strides, int conj,
                         int complex_elem, uint64_t first, uint64_t last, uint32_t* out) {
    if (first >= last) return;
    uint64_t idx[64];
    memset(idx, 0, sizeof(idx));
    uint64_t rem = first;
    for (uint32_t d = rank; d-- > 0;) {
        idx[d] = rem % shape[d];
        rem /= shape[d];
    }
    uint64_t written = first * w;
    for (uint64_t i = first; i < last; ++i) {
        uint64_t e = offset;
        for (uint32_t d = 0; d < rank; ++d) e += idx[d] * strides[d];
        for (uint32_t kw = 0; kw < w; ++kw) {
            uint32_t word = base[e * w + kw];
            if (conj && complex_elem && kw == 1) word ^= 0x80000000u;
            out[written++] = word;
        }
        for (uint32_t d = rank; d-- > 0;) {
            if (++idx[d] < shape[d]) break;
            idx[d] = 0;
        }
    }
}

static uint64_t view_len(uint32_t rank, const uint64_t* shape) {
    uint64_t len = 1;
    for (uint32_t d = 0; d < rank; ++d) len *= shape[d];
    return len;
}

/* Returns the number of words written (len * w). */
uint64_t oracle_gather_words(const uint32_t* base, uint32_t w, uint64_t offset, uint32_t rank,
                             const uint64_t* shape, const uint64_t* strides, int conj,
                             int complex_elem, uint32_t* out) {
    const uint64_t len = view_len(rank, shape);
    gather_range(base, w, offset, rank, shape, strides, conj, complex_elem, 0, len, out);
    return len * w;
}

typedef struct {
    const uint32_t* base;
    uint32_t w, rank;
    uint64_t offset;
    const uint64_t *shape, *strides;
    int conj, complex_elem;
    uint64_t first, last;
    uint32_t* out;
} gather_job;

static void* gather_worker(void* arg) {
    const gather_job* j = (const gather_job*)arg;
    gather_range(j->base, j->w, j->offset, j->rank, j->shape, j->strides, j->conj,
                 j->complex_elem, j->first, j->last, j->out);
    return NULL;
}

/* The same words, with the logical elements split into `threads` contiguous ranges (every
 * word lands where the one-thread form puts it). Returns the words written, or 0 with
 * *failed set when a thread could not be started. */
uint64_t oracle_gather_words_mt(const uint32_t* base, uint32_t w, uint64_t offset,
                                uint32_t rank, const uint64_t* shape, const uint64_t* strides,
                                int conj, int complex_elem, uint32_t* out, int threads,
                                int* failed) {
    const uint64_t len = view_len(rank, shape);
    *failed = 0;
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    if ((uint64_t)threads > len) threads = len ? (int)len : 1;
    gather_job jobs[256];
    pthread_t tids[256];
    for (int t = 0; t < threads; ++t) {
        gather_job* j = &jobs[t];
        j->base = base;
        j->w = w;
        j->rank = rank;
        j->offset = offset;
        j->shape = shape;
        j->strides = strides;
        j->conj = conj;
        j->complex_elem = complex_elem;
        j->first = len * (uint64_t)t / (uint64_t)threads;
        j->last = len * (uint64_t)(t + 1) / (uint64_t)threads;
        j->out = out;
    }
    int started[256] = {0};
    for (int t = 1; t < threads; ++t)
        started[t] = pthread_create(&tids[t], NULL, gather_worker, &jobs[t]) == 0;
    gather_worker(&jobs[0]);
    for (int t = 1; t < threads; ++t) {
        if (started[t]) pthread_join(tids[t], NULL);
        else *failed = 1;
    }
    return *failed ? 0 : len * w;
}

/*
 * The f64 contraction reference of tests/contraction_test.rs:200-268. For every element of
 * C in row-major order of C's labels ("free" labels), with the contracted labels ("sum",
 * in A's label order) running in row-major order:
 *   exact = alpha * sum(a * b) + beta * c0     (f64; alpha = 0 skips A, B; beta = 0 skips C)
 *   magnitude = |alpha| * sum|a * b| + |beta * c0|
 *   index = C's element index
 * Per-label strides are 0 for an operand that does not carry the label.
 */
void oracle_contract_f64(float alpha_f, float beta_f, uint32_t n_free, const uint64_t* free_ext,
                         const int64_t* a_free, const int64_t* b_free, const int64_t* c_free,
                         uint32_t n_sum, const uint64_t* sum_ext, const int64_t* a_sum,
                         const int64_t* b_sum, const float* a, uint64_t a_off, const float* b,
                         uint64_t b_off, const float* c0, uint64_t c_off, double* exact,
                         double* magnitude, uint64_t* index) {
    const double alpha = (double)alpha_f, beta = (double)beta_f;
    uint64_t nf = 1, ns = 1;
    for (uint32_t d = 0; d < n_free; ++d) nf *= free_ext[d];
    for (uint32_t d = 0; d < n_sum; ++d) ns *= sum_ext[d];
    uint64_t fi[64], si[64];
    memset(fi, 0, sizeof(fi));
    for (uint64_t i = 0; i < nf; ++i) {
        int64_t ao = (int64_t)a_off, bo = (int64_t)b_off, co = (int64_t)c_off;
        for (uint32_t d = 0; d < n_free; ++d) {
            ao += (int64_t)fi[d] * a_free[d];
            bo += (int64_t)fi[d] * b_free[d];
            co += (int64_t)fi[d] * c_free[d];
        }
        double sum = 0.0, absum = 0.0;
        if (alpha != 0.0 && ns > 0) {
            memset(si, 0, sizeof(si));
            for (uint64_t s = 0; s < ns; ++s) {
                int64_t ka = 0, kb = 0;
                for (uint32_t d = 0; d < n_sum; ++d) {
                    ka += (int64_t)si[d] * a_sum[d];
                    kb += (int64_t)si[d] * b_sum[d];
                }
                const double p = (double)a[ao + ka] * (double)b[bo + kb];
                sum += p;
                absum += fabs(p);
                for (uint32_t d = n_sum; d-- > 0;) {
                    if (++si[d] < sum_ext[d]) break;
                    si[d] = 0;
                }
            }
            sum *= alpha;
            absum *= fabs(alpha);
        }
        if (beta != 0.0) {
            const double cv = beta * (double)c0[co];
            sum += cv;
            absum += fabs(cv);
        }
        exact[i] = sum;
        magnitude[i] = absum;
        index[i] = (uint64_t)co;
        for (uint32_t d = n_free; d-- > 0;) {
            if (++fi[d] < free_ext[d]) break;
            fi[d] = 0;
        }
    }
}

/* ------------------------------------------------------------------------------------------
 * Backend activation and training ops (crates/cpu/src/lib.rs:297-533,722-729,809-842).
 * Arrays are dense row-major; every expression is the reference's, in its order, one
 * rounding per operation. expf is the C library's, which is what Rust's f32::exp calls on
 * Linux.
 * ---------------------------------------------------------------------------------------- */

/* The f32 spellings of A&S 7.1.26's coefficients and 1/sqrt(2 pi) the reference asserts
 * (crates/cpu/src/lib.rs:846-853): 0.2548296, 0.28449672, 1.4214138, 1.4531521, 1.0614054,
 * 0.3989423. */
static const float ERF_A1 = 0.2548296f;
static const float ERF_A2 = 0.28449672f;
static const float ERF_A3 = 1.4214138f;
static const float ERF_A4 = 1.4531521f;
static const float ERF_A5 = 1.0614054f;
static const float INV_SQRT_2PI = 0.3989423f;
static const float FRAC_1_SQRT_2_F = 0.70710677f; /* std::f32::consts::FRAC_1_SQRT_2 */

/* Bit patterns of the six constants above, for the pinning test. */
void oracle_erf_constants(uint32_t out[6]) {
    const float v[6] = {ERF_A1, ERF_A2, ERF_A3, ERF_A4, ERF_A5, INV_SQRT_2PI};
    memcpy(out, v, sizeof v);
}

/* erf_f32 (crates/cpu/src/lib.rs:811-817). */
static float erf_as(float x) {
    const float sign = signbit(x) ? -1.0f : 1.0f;
    const float a = fabsf(x);
    const float t = 1.0f / (1.0f + 0.3275911f * a);
    const float poly = (((((ERF_A5 * t - ERF_A4) * t) + ERF_A3) * t - ERF_A2) * t + ERF_A1) * t;
    return sign * (1.0f - poly * expf(-a * a));
}

/* gelu_f32 / gelu_prime_f32 (crates/cpu/src/lib.rs:820-829). */
static float gelu_one(float x) {
    const float inner = x * FRAC_1_SQRT_2_F;
    return 0.5f * x * (1.0f + erf_as(inner));
}

static float gelu_prime_one(float x) {
    const float phi = 0.5f * (1.0f + erf_as(x * FRAC_1_SQRT_2_F));
    const float pdf = expf(-0.5f * x * x) * INV_SQRT_2PI;
    return phi + x * pdf;
}

/* CpuBackend::gelu (crates/cpu/src/lib.rs:297-307). */
void oracle_gelu_f32(const float* x, float* y, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) y[i] = gelu_one(x[i]);
}

/* CpuBackend::gelu_backward (crates/cpu/src/lib.rs:309-326): dx = dy * GELU'(pre). */
void oracle_gelu_backward_f32(const float* pre, const float* dy, float* dx, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) dx[i] = dy[i] * gelu_prime_one(pre[i]);
}

/* CpuBackend::add_bias (crates/cpu/src/lib.rs:372-401). y may be x. */
void oracle_add_bias_f32(const float* x, const float* b, float* y, uint64_t rows, uint64_t cols) {
    for (uint64_t r = 0; r < rows; ++r)
        for (uint64_t c = 0; c < cols; ++c) y[r * cols + c] = x[r * cols + c] + b[c];
}

/* CpuBackend::bias_grad (crates/cpu/src/lib.rs:403-435): per column, rows summed in order
 * from +0, then db[j] + s. */
void oracle_bias_grad_f32(const float* dpre, float* db, uint64_t rows, uint64_t cols) {
    if (rows == 0) return;
    for (uint64_t c = 0; c < cols; ++c) {
        float s = 0.0f;
        for (uint64_t r = 0; r < rows; ++r) s += dpre[r * cols + c];
        db[c] = db[c] + s;
    }
}

/* CpuBackend::mse_grad (crates/cpu/src/lib.rs:437-472): one pass in index order. dy may be
 * y. Returns the loss. */
float oracle_mse_grad_f32(const float* y, const float* t, float* dy, uint64_t n) {
    const float nf = (float)n;
    float sum = 0.0f;
    for (uint64_t i = 0; i < n; ++i) {
        const float d = y[i] - t[i];
        sum += d * d;
        dy[i] = (2.0f * d) / nf;
    }
    return sum / nf;
}

/* CpuBackend::sgd_step (crates/cpu/src/lib.rs:474-501). */
void oracle_sgd_step_f32(float* w, float* dw, float lr, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) {
        const float step = lr * dw[i];
        w[i] = w[i] - step;
        dw[i] = 0.0f;
    }
}

/* f32_bits_to_bf16 (crates/cpu/src/lib.rs:725-732) and the bf16 -> f32 widening of
 * CpuBackend::convert (crates/cpu/src/lib.rs:519-527). */
void oracle_f32_to_bf16(const uint32_t* x, uint16_t* y, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) {
        const uint32_t bits = x[i];
        if ((bits & 0x7fffffffu) > 0x7f800000u) {
            y[i] = (uint16_t)((bits >> 16) | 0x0040u);
        } else {
            const uint32_t lsb = (bits >> 16) & 1u;
            y[i] = (uint16_t)((bits + 0x7fffu + lsb) >> 16);
        }
    }
}

void oracle_bf16_to_f32(const uint16_t* x, uint32_t* y, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) y[i] = (uint32_t)x[i] << 16;
}

/* ---- CpuBackend::gemm on F16 / BF16 tensors -------------------------------------------
 * crates/cpu loads and stores 16-bit elements through the `half` crate, version 2.7.1
 * (pinned =2.7.1 by crates/cpu/Cargo.toml:14; not vendored under the reference), with its
 * `*_const` conversions (crates/cpu/src/lib.rs:694-720). Restated from the crate's published
 * f16 <-> f32 algorithm:
 *   f16 -> f32: exact; a NaN keeps sign and payload (shifted up 13) and gets the quiet bit.
 *   f32 -> f16: round to nearest even on the f32 bits; halves of the subnormal range kept,
 *     values from 65520 up overflow to infinity, below 2^-25 (and ties at 2^-25) to zero;
 *     a NaN keeps the sign and the top ten payload bits and gets the quiet bit (0x0200).
 *   bf16 <-> f32: the high half of the f32 bits, rounded to nearest even, NaN | 0x0040,
 *     which is oracle_f32_to_bf16 above. */
static float f16_bits_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (man ? 0x00400000u | (man << 13) : 0u);
    } else if (exp != 0) {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    } else if (man == 0) {
        bits = sign;
    } else {  /* subnormal: man * 2^-24, normalised */
        int e = -14;
        uint32_t m = man;
        while (!(m & 0x400u)) { m <<= 1; --e; }
        bits = sign | ((uint32_t)(e + 127) << 23) | ((m & 0x3ffu) << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t oracle_f32_to_f16_bits(uint32_t x) {
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t exp = x & 0x7f800000u, man = x & 0x007fffffu;
    if (exp == 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (man ? 0x0200u | (man >> 13) : 0u));
    const int half_exp = (int)(exp >> 23) - 127 + 15;
    if (half_exp >= 0x1f) return (uint16_t)(sign | 0x7c00u);
    if (half_exp <= 0) {
        if (14 - half_exp > 24) return (uint16_t)sign;
        const uint32_t full = man | 0x00800000u;
        uint32_t half_man = full >> (14 - half_exp);
        const uint32_t round_bit = 1u << (13 - half_exp);
        /* ties to even: the round bit and any lower bit or the kept least significant bit */
        if ((full & round_bit) && (full & (3u * round_bit - 1u))) ++half_man;
        return (uint16_t)(sign | half_man);
    }
    uint32_t out = sign | ((uint32_t)half_exp << 10) | (man >> 13);
    if ((man & 0x1000u) && (man & 0x2fffu)) ++out;  /* a carry runs into the exponent */
    return (uint16_t)out;
}

void oracle_f32_to_f16(const uint32_t* x, uint16_t* y, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) y[i] = oracle_f32_to_f16_bits(x[i]);
}

void oracle_f16_to_f32(const uint16_t* x, float* y, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) y[i] = f16_bits_to_f32(x[i]);
}

static float widen16(int kind, uint16_t h) {
    if (kind == 0) return f16_bits_to_f32(h);
    const uint32_t bits = (uint32_t)h << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static uint16_t narrow16(int kind, float v) {
    uint32_t bits;
    uint16_t out;
    memcpy(&bits, &v, 4);
    if (kind == 0) return oracle_f32_to_f16_bits(bits);
    oracle_f32_to_bf16(&bits, &out, 1);
    return out;
}

/*
 * CpuBackend::gemm with dtype F16 (kind 0) or BF16 (kind 1): crates/cpu/src/lib.rs:270-291
 * hands `accumulate` (:664-691) loaders that widen each element to f32 and a store that
 * rounds the f32 accumulator to 16 bits, so for every (row, col) in row-major order
 *   acc = (beta == 0) ? +0 : beta * widen(C[row, col])              (C unread when beta is 0)
 *   if (alpha != 0) for inner in 0..k: acc += (alpha * widen(A[row, inner])) * widen(B[inner, col])
 *   C[row, col] = narrow(acc)
 * with every f32 multiply and add rounded on its own. Strides in elements.
 */
void oracle_gemm_seq_16(int kind, uint64_t m, uint64_t n, uint64_t k, float alpha, float beta,
                        const uint16_t* a, int64_t a_rs, int64_t a_cs,
                        const uint16_t* b, int64_t b_rs, int64_t b_cs,
                        uint16_t* c, int64_t c_rs, int64_t c_cs) {
    for (uint64_t row = 0; row < m; ++row) {
        for (uint64_t col = 0; col < n; ++col) {
            uint16_t* out = c + (int64_t)row * c_rs + (int64_t)col * c_cs;
            float acc = (beta == 0.0f) ? 0.0f : beta * widen16(kind, *out);
            if (alpha != 0.0f) {
                for (uint64_t inner = 0; inner < k; ++inner) {
                    const float t = alpha * widen16(kind, a[(int64_t)row * a_rs + (int64_t)inner * a_cs]);
                    const float p = t * widen16(kind, b[(int64_t)inner * b_rs + (int64_t)col * b_cs]);
                    acc = acc + p;
                }
            }
            *out = narrow16(kind, acc);
        }
    }
}

/*
 * lava_oracle.c -- CPU restatement of Lava.jl's cooperative-matrix compute path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker, never the thing measured
 * or shipped: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it.  The product path (liblava_hip.so) never links it and never
 * falls back to it.
 *
 * What each function restates (paths relative to the Lava.jl source tree):
 *
 *   oracle_gemm_rows       D = A*B + 0 of `coopmat_muladd` / `muladd(a, b, zero(...))`
 *                          (src/vocabulary/coopmat.jl:196-203), over row/column-major
 *                          operands as `coopmat_load(..., Val(rowmajor))` addresses them
 *                          (src/vocabulary/coopmat.jl:124-140, src/compiler/spirv/
 *                          coopmat.jl:664-744), in fp64 on the fp16/bf16-rounded inputs.
 *   oracle_gemm_f32acc     The same product accumulated in fp32, the accumulator type of
 *                          `AcceleratedMatrix{Float32,...,Accumulator}`; used as the CPU
 *                          baseline (docs/src/device.md:81-88 tile loop).
 *   oracle_gemm_i8_rows    int8 x int8 -> int32 with A, B, C and Result all signed
 *                          (src/compiler/spirv/coopmat.jl:115-151; test/spirv/
 *                          test_coopmat_int8.jl:25-69), exact in int64.
 *   oracle_gemm_u8_rows    uint8 x uint8 -> uint32, no signedness operands
 *                          (test/spirv/test_coopmat_int8.jl:71-98).
 *   oracle_w8a16_rows      Y = (X * float(W)) .* s[col]: the per-element dequant callback
 *                          `f(row, col, e, scales...)` of `coopmat_perelement`
 *                          (src/device/coopmat_intrinsics.jl:535-628).
 *   oracle_attn_rows       O = softmax(Q K^T * scale + causal) V over (E,L,H,B) tensors,
 *                          head dim fastest (src/device/tensor_intrinsics.jl:279-281),
 *                          the flash form of src/device/coopmat_intrinsics.jl:638-720.
 *   oracle_dot4x8          src/vocabulary/vocabulary.jl:31-35.
 *   oracle_f32_to_f16      RNE narrowing, src/compiler/passes/exact_narrowing.jl:31-36.
 *   oracle_f32_to_bf16     RNE narrowing to bfloat16 (no Lava counterpart: the coopmat
 *                          component table has no bf16, src/device/coopmat_intrinsics.jl:16-19).
 *   oracle_rng_u64 / oracle_fill_*
 *                          the seeded counter-based input generator (splitmix64 of
 *                          (seed, index)); the same definition is implemented on the
 *                          device by liblava_hip.so's fill kernels.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* Generator                                                                 */
/* ------------------------------------------------------------------------ */

/* splitmix64 (Steele, Lea, Flood 2014; Vigna's public-domain constants) applied to
 * a counter: z = seed * 0xD1B54A32D192ED03 + (i + 1) * 0x9E3779B97F4A7C15, then the
 * splitmix64 finaliser. */
uint64_t oracle_rng_u64(uint64_t seed, uint64_t i) {
    uint64_t z = seed * 0xD1B54A32D192ED03ull + (i + 1ull) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* IEEE binary32 -> binary16, round to nearest even, NaN stays NaN (quiet),
 * overflow to +-Inf.  Written from the format definitions. */
uint16_t oracle_f32_to_f16(float f) {
    uint32_t x = f32_bits(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    if (ax == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
    int32_t e = (int32_t)(ax >> 23) - 127;          /* unbiased exponent */
    uint32_t mant = (ax & 0x7fffffu) | (ax >= 0x00800000u ? 0x800000u : 0u);
    if (ax < 0x00800000u) e = -126;                  /* f32 subnormal */
    if (e > 15) return (uint16_t)(sign | 0x7c00u);
    /* value = mant * 2^(e-23).  Target: half with 10 fraction bits.
       For normal half: e >= -14, shift = 13.  Subnormal half: unit 2^-24. */
    int32_t shift;
    uint32_t hexp;
    if (e >= -14) { shift = 13; hexp = (uint32_t)(e + 15); }
    else { shift = 13 + (-14 - e); hexp = 0; }
    if (shift > 24 + 1) return (uint16_t)sign;       /* rounds to zero */
    uint32_t q = mant >> shift;
    uint32_t rem = mant & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    uint32_t out;
    if (hexp == 0) {
        out = q;                                      /* may carry into the smallest normal */
    } else {
        /* q has the implicit bit at 1<<10 */
        out = (hexp << 10) + (q - 0x400u);
        if (q == 0x800u) out = ((hexp + 1u) << 10);   /* mantissa overflow */
    }
    if (out >= 0x7c00u) out = 0x7c00u;
    return (uint16_t)(sign | out);
}

float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0) {
        float v = (float)m * 5.9604644775390625e-08f; /* 2^-24 */
        return sign ? -v : v;
    }
    if (e == 31) return bits_f32(sign | 0x7f800000u | (m << 13));
    return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
}

/* IEEE binary32 -> bfloat16 (upper 16 bits), round to nearest even. */
uint16_t oracle_f32_to_bf16(float f) {
    uint32_t x = f32_bits(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    uint32_t lsb = (x >> 16) & 1u;
    x += 0x7fffu + lsb;
    return (uint16_t)(x >> 16);
}

float oracle_bf16_to_f32(uint16_t b) { return bits_f32((uint32_t)b << 16); }

/* Uniform[a, b]: k = top 24 bits of the draw; v = fl32(a + (b - a) * k * 2^-24),
 * the sum computed in binary64 and rounded once to binary32. */
static inline float uniform_f32(uint64_t seed, uint64_t i, double a, double b) {
    uint64_t k = oracle_rng_u64(seed, i) >> 40;
    return (float)(a + (b - a) * ((double)k * 5.9604644775390625e-08));
}

/* normal(0,1): Box-Muller on the two 32-bit halves of one draw,
 * u1 = (hi + 0.5) 2^-32, u2 = (lo + 0.5) 2^-32, n = sqrt(-2 ln u1) cos(2 pi u2),
 * in binary64, rounded once to binary32. */
static inline float normal_f32(uint64_t seed, uint64_t i) {
    uint64_t z = oracle_rng_u64(seed, i);
    double u1 = ((double)(z >> 32) + 0.5) * 2.3283064365386963e-10;
    double u2 = ((double)(z & 0xffffffffull) + 0.5) * 2.3283064365386963e-10;
    return (float)(sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2));
}

/* dtype codes shared with the product library */
enum { DT_F16 = 0, DT_BF16 = 1, DT_F32 = 2, DT_I8 = 3, DT_U8 = 4, DT_I32 = 5 };

void oracle_fill_uniform(void* out, int dtype, int64_t n, uint64_t seed, double a, double b) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        float v = uniform_f32(seed, (uint64_t)i, a, b);
        if (dtype == DT_F16) ((uint16_t*)out)[i] = oracle_f32_to_f16(v);
        else if (dtype == DT_BF16) ((uint16_t*)out)[i] = oracle_f32_to_bf16(v);
        else ((float*)out)[i] = v;
    }
}

void oracle_fill_normal(void* out, int dtype, int64_t n, uint64_t seed) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        float v = normal_f32(seed, (uint64_t)i);
        if (dtype == DT_F16) ((uint16_t*)out)[i] = oracle_f32_to_f16(v);
        else if (dtype == DT_BF16) ((uint16_t*)out)[i] = oracle_f32_to_bf16(v);
        else ((float*)out)[i] = v;
    }
}

/* int8 over [-128, 127]: the top byte of the draw.
 * int8 over [-127, 127]: (draw >> 32) mod 255 - 127. */
void oracle_fill_i8(int8_t* out, int64_t n, uint64_t seed, int symmetric) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        uint64_t z = oracle_rng_u64(seed, (uint64_t)i);
        out[i] = symmetric ? (int8_t)((int)((z >> 32) % 255u) - 127) : (int8_t)(uint8_t)(z >> 56);
    }
}

/* ------------------------------------------------------------------------ */
/* Element access                                                            */
/* ------------------------------------------------------------------------ */

static inline double load_fp(const void* p, int dtype, int64_t idx) {
    switch (dtype) {
    case DT_F16: return (double)oracle_f16_to_f32(((const uint16_t*)p)[idx]);
    case DT_BF16: return (double)oracle_bf16_to_f32(((const uint16_t*)p)[idx]);
    case DT_F32: return (double)((const float*)p)[idx];
    case DT_I8: return (double)((const int8_t*)p)[idx];
    default: return 0.0;
    }
}

/* Layout flags: bit0 A row-major, bit1 B row-major, bit2 C row-major
 * (else column-major, Julia's default; src/device/devicearray.jl:138-174). */
static inline int64_t a_index(int64_t i, int64_t k, int64_t lda, uint32_t layout) {
    return (layout & 1u) ? i * lda + k : k * lda + i;
}
static inline int64_t b_index(int64_t k, int64_t j, int64_t ldb, uint32_t layout) {
    return (layout & 2u) ? k * ldb + j : j * ldb + k;
}

/* ------------------------------------------------------------------------ */
/* GEMM                                                                      */
/* ------------------------------------------------------------------------ */

/* C[rows[r], j] for j < N, fp64 accumulate over the exactly-decoded inputs.
 * out is nrows x N, row-major. */
void oracle_gemm_rows(const void* A, int adt, const void* B, int bdt,
                      int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                      uint32_t layout, const int64_t* rows, int64_t nrows, double* out) {
    (void)M;
    double* bcol = (double*)malloc(sizeof(double) * (size_t)K * (size_t)N);
    /* decode B once, k-fastest per column */
#pragma omp parallel for schedule(static)
    for (int64_t j = 0; j < N; ++j)
        for (int64_t k = 0; k < K; ++k) bcol[j * K + k] = load_fp(B, bdt, b_index(k, j, ldb, layout));
#pragma omp parallel
    {
        double* arow = (double*)malloc(sizeof(double) * (size_t)K);
#pragma omp for schedule(dynamic, 1)
        for (int64_t r = 0; r < nrows; ++r) {
            int64_t i = rows[r];
            for (int64_t k = 0; k < K; ++k) arow[k] = load_fp(A, adt, a_index(i, k, lda, layout));
            for (int64_t j = 0; j < N; ++j) {
                const double* bc = bcol + j * K;
                double s = 0.0;
                for (int64_t k = 0; k < K; ++k) s += arow[k] * bc[k];
                out[r * N + j] = s;
            }
        }
        free(arow);
    }
    free(bcol);
}

/* The CPU baseline: the same product with fp32 accumulation, all host threads.
 * Computes rows [0, nrows) of C (row-major, ldc = N) into out. */
void oracle_gemm_f32acc(const void* A, int adt, const void* B, int bdt,
                        int64_t N, int64_t K, int64_t lda, int64_t ldb, uint32_t layout,
                        int64_t nrows, float* out) {
    float* bcol = (float*)malloc(sizeof(float) * (size_t)K * (size_t)N);
#pragma omp parallel for schedule(static)
    for (int64_t j = 0; j < N; ++j)
        for (int64_t k = 0; k < K; ++k) bcol[j * K + k] = (float)load_fp(B, bdt, b_index(k, j, ldb, layout));
#pragma omp parallel
    {
        float* arow = (float*)malloc(sizeof(float) * (size_t)K);
#pragma omp for schedule(dynamic, 1)
        for (int64_t i = 0; i < nrows; ++i) {
            for (int64_t k = 0; k < K; ++k) arow[k] = (float)load_fp(A, adt, a_index(i, k, lda, layout));
            for (int64_t j = 0; j < N; ++j) {
                const float* bc = bcol + j * K;
                float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f, s4 = 0.f, s5 = 0.f, s6 = 0.f, s7 = 0.f;
                int64_t k = 0;
                for (; k + 8 <= K; k += 8) {
                    s0 += arow[k] * bc[k];         s1 += arow[k + 1] * bc[k + 1];
                    s2 += arow[k + 2] * bc[k + 2]; s3 += arow[k + 3] * bc[k + 3];
                    s4 += arow[k + 4] * bc[k + 4]; s5 += arow[k + 5] * bc[k + 5];
                    s6 += arow[k + 6] * bc[k + 6]; s7 += arow[k + 7] * bc[k + 7];
                }
                for (; k < K; ++k) s0 += arow[k] * bc[k];
                out[i * N + j] = ((s0 + s1) + (s2 + s3)) + ((s4 + s5) + (s6 + s7));
            }
        }
        free(arow);
    }
    free(bcol);
}

/* int8 x int8 -> int32 (signed) or uint8 x uint8 -> uint32, exact (int64 sums,
 * then the two's-complement wrap to 32 bits that a 32-bit accumulator performs). */
static void gemm_int_rows(const void* A, const void* B, int is_signed,
                          int64_t N, int64_t K, int64_t lda, int64_t ldb, uint32_t layout,
                          const int64_t* rows, int64_t nrows, int32_t* out) {
    int64_t* bcol = (int64_t*)malloc(sizeof(int64_t) * (size_t)K * (size_t)N);
#pragma omp parallel for schedule(static)
    for (int64_t j = 0; j < N; ++j)
        for (int64_t k = 0; k < K; ++k) {
            int64_t idx = b_index(k, j, ldb, layout);
            bcol[j * K + k] = is_signed ? (int64_t)((const int8_t*)B)[idx] : (int64_t)((const uint8_t*)B)[idx];
        }
#pragma omp parallel
    {
        int64_t* arow = (int64_t*)malloc(sizeof(int64_t) * (size_t)K);
#pragma omp for schedule(dynamic, 1)
        for (int64_t r = 0; r < nrows; ++r) {
            int64_t i = rows[r];
            for (int64_t k = 0; k < K; ++k) {
                int64_t idx = a_index(i, k, lda, layout);
                arow[k] = is_signed ? (int64_t)((const int8_t*)A)[idx] : (int64_t)((const uint8_t*)A)[idx];
            }
            for (int64_t j = 0; j < N; ++j) {
                const int64_t* bc = bcol + j * K;
                int64_t s = 0;
                for (int64_t k = 0; k < K; ++k) s += arow[k] * bc[k];
                out[r * N + j] = (int32_t)(uint32_t)(uint64_t)s;
            }
        }
        free(arow);
    }
    free(bcol);
}

void oracle_gemm_i8_rows(const int8_t* A, const int8_t* B, int64_t N, int64_t K, int64_t lda,
                         int64_t ldb, uint32_t layout, const int64_t* rows, int64_t nrows,
                         int32_t* out) {
    gemm_int_rows(A, B, 1, N, K, lda, ldb, layout, rows, nrows, out);
}

void oracle_gemm_u8_rows(const uint8_t* A, const uint8_t* B, int64_t N, int64_t K, int64_t lda,
                         int64_t ldb, uint32_t layout, const int64_t* rows, int64_t nrows,
                         uint32_t* out) {
    gemm_int_rows(A, B, 0, N, K, lda, ldb, layout, rows, nrows, (int32_t*)out);
}

/* W8A16: X (M x K fp16, row-major, ldx), W (K x N int8, row-major, ldw),
 * s (N fp16), Y[r, j] = s[j] * sum_k X[i,k] W[k,j], fp64. */
void oracle_w8a16_rows(const uint16_t* X, const int8_t* W, const uint16_t* s,
                       int64_t N, int64_t K, int64_t ldx, int64_t ldw,
                       const int64_t* rows, int64_t nrows, double* out) {
#pragma omp parallel for schedule(static)
    for (int64_t j = 0; j < N; ++j) {
        double sc = (double)oracle_f16_to_f32(s[j]);
        for (int64_t r = 0; r < nrows; ++r) {
            const uint16_t* x = X + rows[r] * ldx;
            double acc = 0.0;
            for (int64_t k = 0; k < K; ++k)
                acc += (double)oracle_f16_to_f32(x[k]) * (double)W[k * ldw + j];
            out[r * N + j] = acc * sc;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Attention                                                                 */
/* ------------------------------------------------------------------------ */

/* Q, K, V are fp16 tensors with element (e, l, h, b) at
 * e*st[0] + l*st[1] + h*st[2] + b*st[3] (the (E,L,H,B) layout, head dim fastest when
 * st[0] == 1).  For one (b, h) and the query rows `qrows`, out[r, e] (nq x D, fp64)
 * = sum_j softmax_j(scale * q.k_j, j <= q if causal) v_j[e]. */
void oracle_attn_rows(const uint16_t* Q, const uint16_t* K, const uint16_t* V,
                      int64_t S, int64_t D, const int64_t* st, double scale, int causal,
                      int64_t b, int64_t h, const int64_t* qrows, int64_t nq, double* out) {
    int64_t base = h * st[2] + b * st[3];
    double* kd = (double*)malloc(sizeof(double) * (size_t)(S * D));
    double* vd = (double*)malloc(sizeof(double) * (size_t)(S * D));
#pragma omp parallel for schedule(static)
    for (int64_t l = 0; l < S; ++l)
        for (int64_t e = 0; e < D; ++e) {
            kd[l * D + e] = (double)oracle_f16_to_f32(K[base + e * st[0] + l * st[1]]);
            vd[l * D + e] = (double)oracle_f16_to_f32(V[base + e * st[0] + l * st[1]]);
        }
#pragma omp parallel
    {
        double* sc = (double*)malloc(sizeof(double) * (size_t)S);
        double* q = (double*)malloc(sizeof(double) * (size_t)D);
#pragma omp for schedule(dynamic, 1)
        for (int64_t r = 0; r < nq; ++r) {
            int64_t i = qrows[r];
            for (int64_t e = 0; e < D; ++e) q[e] = (double)oracle_f16_to_f32(Q[base + e * st[0] + i * st[1]]);
            int64_t nk = causal ? i + 1 : S;
            double mx = -INFINITY;
            for (int64_t j = 0; j < nk; ++j) {
                double s = 0.0;
                for (int64_t e = 0; e < D; ++e) s += q[e] * kd[j * D + e];
                s *= scale;
                sc[j] = s;
                if (s > mx) mx = s;
            }
            double den = 0.0;
            for (int64_t j = 0; j < nk; ++j) { sc[j] = exp(sc[j] - mx); den += sc[j]; }
            for (int64_t e = 0; e < D; ++e) {
                double acc = 0.0;
                for (int64_t j = 0; j < nk; ++j) acc += sc[j] * vd[j * D + e];
                out[r * D + e] = acc / den;
            }
        }
        free(sc);
        free(q);
    }
    free(kd);
    free(vd);
}

/* ------------------------------------------------------------------------ */
/* Scalar vocabulary                                                         */
/* ------------------------------------------------------------------------ */

/* dot4x8(a, b) = sum_i sext(byte_i a) * sext(byte_i b)  (vocabulary.jl:31-35) */
int32_t oracle_dot4x8(uint32_t a, uint32_t b) {
    int32_t s = 0;
    for (int i = 0; i < 4; ++i) s += (int32_t)(int8_t)(uint8_t)(a >> (8 * i)) * (int32_t)(int8_t)(uint8_t)(b >> (8 * i));
    return s;
}

void oracle_dot4x8_array(const uint32_t* a, const uint32_t* b, int32_t* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = oracle_dot4x8(a[i], b[i]);
}

void oracle_f32_to_f16_array(const float* x, uint16_t* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = oracle_f32_to_f16(x[i]);
}

void oracle_f32_to_bf16_array(const float* x, uint16_t* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = oracle_f32_to_bf16(x[i]);
}

int oracle_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

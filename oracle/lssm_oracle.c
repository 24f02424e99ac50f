/*
 * lssm_oracle.c — CPU restatement of lite-ssm's Metal kernels.
 *
 * TEST INFRASTRUCTURE ONLY: the parity oracle and the timed CPU baseline.
 * Nothing in the product library links or calls this file.
 *
 * Each function names the reference file:line whose arithmetic it restates.
 * Reductions are accumulated in double (the exact value that the reference's
 * fp32 reductions approximate in an unspecified order); elementwise math is
 * fp32; r() rounds to the activation dtype (RNE) wherever the reference
 * stores a `half`.
 */
#include "lssm_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------- */
/* conversions                                                                */
/* ------------------------------------------------------------------------- */
uint16_t orc_f2h(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t a = x & 0x7fffffffu;
    if (a >= 0x7f800000u) {                       /* inf / nan */
        if (a == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu));
    }
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);   /* >= 65520 -> inf */
    if (a < 0x38800000u) {                        /* below 2^-14: half subnormal */
        if (a <= 0x33000000u) return (uint16_t)sign;            /* <= 2^-25 -> 0 */
        uint32_t e = a >> 23;
        uint32_t m = (a & 0x7fffffu) | 0x800000u;
        uint32_t sh = 126u - e;                   /* 14..24 */
        uint32_t q = m >> sh;
        uint32_t rem = m & ((1u << sh) - 1u);
        uint32_t hlf = 1u << (sh - 1u);
        if (rem > hlf || (rem == hlf && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t r = a + 0xfffu + ((a >> 13) & 1u);
    r -= 0x38000000u;
    return (uint16_t)(sign | (r >> 13));
}

float orc_h2f(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t f;
    if (e == 0) {
        if (m == 0) {
            f = sign;
        } else {
            float v = (float)m * (1.0f / 16777216.0f);   /* m * 2^-24, exact */
            memcpy(&f, &v, 4);
            f |= sign;
        }
    } else if (e == 31) {
        f = sign | 0x7f800000u | (m << 13);
    } else {
        f = sign | ((e + 112u) << 23) | (m << 13);
    }
    float out;
    memcpy(&out, &f, 4);
    return out;
}

uint16_t orc_f2b(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    x += 0x7fffu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

float orc_b2f(uint16_t b) {
    uint32_t x = (uint32_t)b << 16;
    float f;
    memcpy(&f, &x, 4);
    return f;
}

static inline float ld(const void* p, size_t i, int dt) {
    if (dt == LSSM_F16) return orc_h2f(((const uint16_t*)p)[i]);
    if (dt == LSSM_BF16) return orc_b2f(((const uint16_t*)p)[i]);
    return ((const float*)p)[i];
}

static inline void st(void* p, size_t i, int dt, float v) {
    if (dt == LSSM_F16) ((uint16_t*)p)[i] = orc_f2h(v);
    else if (dt == LSSM_BF16) ((uint16_t*)p)[i] = orc_f2b(v);
    else ((float*)p)[i] = v;
}

/* r(): round to the activation dtype */
static inline float rnd(float v, int dt) {
    if (dt == LSSM_F16) return orc_h2f(orc_f2h(v));
    if (dt == LSSM_BF16) return orc_b2f(orc_f2b(v));
    return v;
}

static inline size_t esz(int dt) { return dt == LSSM_F32 ? 4 : 2; }

void orc_f32_to_act(const float* in, void* out, size_t n, int dt) {
    for (size_t i = 0; i < n; ++i) st(out, i, dt, in[i]);
}
void orc_act_to_f32(const void* in, float* out, size_t n, int dt) {
    for (size_t i = 0; i < n; ++i) out[i] = ld(in, i, dt);
}

static inline float silu_f(float v) { return v / (1.0f + expf(-v)); }   /* common.metal:48-50 */
static inline float softplus_f(float v) { return (v > 20.0f) ? v : logf(1.0f + expf(v)); } /* ssd_step.metal:26-28 */
static inline float clampf_(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }

int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
void orc_set_num_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

/* Summation of the linears' dot products: double (the default, as close to
 * exact as the oracle gets) or float32 in sixteen interleaved partial sums.
 * The reference's kernels accumulate in fp32 in their own order
 * (linear.metal:100-108, 463-473), so both are faithful restatements; the
 * float32 mode exists to measure how far two such restatements part over a
 * whole model, which is the yardstick for the GPU path's whole-model drift. */
static int g_accum_f32 = 0;
void orc_set_accum(int f32) { g_accum_f32 = f32 != 0; }
int orc_accum(void) { return g_accum_f32; }

/* ------------------------------------------------------------------------- */
/* weight formats                                                             */
/* ------------------------------------------------------------------------- */
size_t orc_wfmt_group(int wfmt) {
    switch (wfmt) {
        case LSSM_W_Q4_B32: return 32;   /* ssm_format.hpp:43 */
        case LSSM_W_Q4_G64: return 64;
        case LSSM_W_Q8_G32: return 32;
        default: return 0;
    }
}

size_t orc_packed_nbytes(int wfmt, size_t N, size_t K, int act) {
    size_t numel = N * K;
    switch (wfmt) {
        case LSSM_W_Q4_B32: return numel / 2 + (numel / 32) * 2;   /* ssm_format.hpp:64-69 */
        case LSSM_W_Q4_G64: return numel / 2 + (numel / 64) * 2;
        case LSSM_W_Q8_G32: return numel + (numel / 32) * 2;
        default: return numel * esz(act);
    }
}

static inline int q_at(const uint8_t* packed, size_t row_bytes, uint32_t n, uint32_t k, int wfmt) {
    if (wfmt == LSSM_W_Q8_G32) return (int)(int8_t)packed[(size_t)n * row_bytes + k];
    /* linear.metal:47-61: byte = packed[n*K/2 + k/2]; low nibble for even k */
    uint8_t b = packed[(size_t)n * row_bytes + (k >> 1)];
    uint32_t nib = (k & 1u) ? (uint32_t)(b >> 4) : (uint32_t)(b & 0x0fu);
    return (nib < 8u) ? (int)nib : (int)nib - 16;
}

/* Dequantize row n into fp32 (exact: |q| <= 128 times an fp16 scale). */
static void deq_row(const void* w, const void* s, float* out, uint32_t n, uint32_t K,
                    int wfmt, int act) {
    if (wfmt == LSSM_W_DENSE) {
        for (uint32_t k = 0; k < K; ++k) out[k] = ld(w, (size_t)n * K + k, act);
        return;
    }
    const uint8_t* packed = (const uint8_t*)w;
    const uint16_t* scales = (const uint16_t*)s;
    size_t row_bytes = (wfmt == LSSM_W_Q8_G32) ? K : K / 2;
    uint32_t G = (uint32_t)orc_wfmt_group(wfmt);
    uint32_t gpr = K / G;
    const uint8_t* row = packed + (size_t)n * row_bytes;
    for (uint32_t g = 0; g < gpr; ++g) {
        const float sc = orc_h2f(scales[(size_t)n * gpr + g]);
        float* o = out + (size_t)g * G;
        if (wfmt == LSSM_W_Q8_G32) {
            for (uint32_t i = 0; i < G; ++i) o[i] = (float)(int8_t)row[(size_t)g * G + i] * sc;
        } else {
            /* linear.metal:47-61: low nibble = even k, two's complement 4-bit */
            const uint8_t* b = row + (size_t)g * G / 2;
            for (uint32_t i = 0; i < G / 2; ++i) {
                /* sign-extend each nibble: shift it to the top of a signed byte */
                const int lo = (int8_t)(uint8_t)(b[i] << 4) >> 4, hi = (int8_t)b[i] >> 4;
                o[2 * i] = (float)lo * sc;
                o[2 * i + 1] = (float)hi * sc;
            }
        }
    }
}

void orc_dequant(const void* w, const void* s, float* out, uint32_t N, uint32_t K, int wfmt,
                 int act) {
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < (int64_t)N; ++n) deq_row(w, s, out + (size_t)n * K, (uint32_t)n, K, wfmt, act);
}

/* tools/export_mamba2.py:68-103: per group absmax (clamp >= 1e-12) / qmax in
 * fp32; q = round_half_even(w / scale_f32) clamped to [qmin, qmax]; the scale is
 * stored as fp16.  qmax = 7 (int4) or 127 (int8). */
void orc_quantize(const float* w, uint32_t N, uint32_t K, int wfmt, uint8_t* packed,
                  uint16_t* scales) {
    uint32_t G = (uint32_t)orc_wfmt_group(wfmt);
    int is8 = (wfmt == LSSM_W_Q8_G32);
    float qmax = is8 ? 127.0f : 7.0f;
    float qmin = is8 ? -128.0f : -8.0f;
    uint32_t gpr = K / G;
    size_t row_bytes = is8 ? K : K / 2;
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < (int64_t)N; ++n) {
        for (uint32_t g = 0; g < gpr; ++g) {
            const float* blk = w + (size_t)n * K + (size_t)g * G;
            float amax = 0.0f;
            for (uint32_t i = 0; i < G; ++i) {
                float a = fabsf(blk[i]);
                if (a > amax) amax = a;
            }
            if (amax < 1e-12f) amax = 1e-12f;
            float scale = amax / qmax;
            scales[(size_t)n * gpr + g] = orc_f2h(scale);
            for (uint32_t i = 0; i < G; ++i) {
                float q = rintf(blk[i] / scale);
                q = clampf_(q, qmin, qmax);
                int qi = (int)q;
                uint32_t k = g * G + i;
                if (is8) {
                    packed[(size_t)n * row_bytes + k] = (uint8_t)(int8_t)qi;
                } else {
                    uint8_t* b = &packed[(size_t)n * row_bytes + (k >> 1)];
                    uint8_t nib = (uint8_t)(qi & 0x0f);
                    if (k & 1u) *b = (uint8_t)((*b & 0x0fu) | (nib << 4));
                    else *b = (uint8_t)((*b & 0xf0u) | nib);
                }
            }
        }
    }
}

/* ------------------------------------------------------------------------- */
/* kernels                                                                    */
/* ------------------------------------------------------------------------- */
/* norm.metal:52-79 — y = r(x * w * rsqrt(sum(x^2)/dim + eps)) */
void orc_rmsnorm(const void* x, const void* w, void* y, uint32_t rows, uint32_t dim, float eps,
                 int act) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < (int64_t)rows; ++r) {
        size_t base = (size_t)r * dim;
        double ss = 0.0;
        for (uint32_t i = 0; i < dim; ++i) {
            double v = ld(x, base + i, act);
            ss += v * v;
        }
        float rrms = 1.0f / sqrtf((float)ss / (float)dim + eps);
        for (uint32_t i = 0; i < dim; ++i) {
            float v = ld(x, base + i, act) * ld(w, i, act) * rrms;
            st(y, base + i, act, v);
        }
    }
}

/* Sum of a[k] * b[k] in double.  Sixteen independent partial sums (the order
 * in which double additions happen is immaterial at every tolerance the
 * oracle is used with) keep the loop vectorised instead of latency-bound. */
typedef double v4d __attribute__((vector_size(32)));
static inline v4d ld4(const double* p) {
    v4d v;
    memcpy(&v, p, sizeof(v));
    return v;
}
static inline double hsum4(v4d v) { return (v[0] + v[1]) + (v[2] + v[3]); }

/* Sums of w[k] * x_r[k] in double for rows x_0..x_3 of x (row stride K), with
 * independent partial sums: the order of double additions is immaterial at
 * every tolerance the oracle is used with, and this keeps the loop vectorised
 * with the weight row loaded once for four rows. */
static void dot4_f64(const double* w, const double* x, uint32_t K, double* out) {
    const double *x0 = x, *x1 = x + K, *x2 = x + 2 * (size_t)K, *x3 = x + 3 * (size_t)K;
    v4d a0 = {0, 0, 0, 0}, a1 = a0, a2 = a0, a3 = a0, b0 = a0, b1 = a0, b2 = a0, b3 = a0;
    uint32_t k = 0;
    for (; k + 8 <= K; k += 8) {
        const v4d w0 = ld4(w + k), w1 = ld4(w + k + 4);
        a0 += w0 * ld4(x0 + k); b0 += w1 * ld4(x0 + k + 4);
        a1 += w0 * ld4(x1 + k); b1 += w1 * ld4(x1 + k + 4);
        a2 += w0 * ld4(x2 + k); b2 += w1 * ld4(x2 + k + 4);
        a3 += w0 * ld4(x3 + k); b3 += w1 * ld4(x3 + k + 4);
    }
    out[0] = hsum4(a0 + b0); out[1] = hsum4(a1 + b1); out[2] = hsum4(a2 + b2); out[3] = hsum4(a3 + b3);
    for (; k < K; ++k) {
        out[0] += w[k] * x0[k]; out[1] += w[k] * x1[k]; out[2] += w[k] * x2[k]; out[3] += w[k] * x3[k];
    }
}

/* float32 sums of w[k] * x[k], sixteen partial sums added pairwise */
static float dot1_f32(const double* w, const double* x, uint32_t K) {
    float p[16] = {0};
    uint32_t k = 0;
    for (; k + 16 <= K; k += 16)
        for (int j = 0; j < 16; ++j) p[j] = fmaf((float)w[k + j], (float)x[k + j], p[j]);
    for (int w2 = 8; w2 >= 1; w2 >>= 1)
        for (int j = 0; j < w2; ++j) p[j] += p[j + w2];
    float t = p[0];
    for (; k < K; ++k) t = fmaf((float)w[k], (float)x[k], t);
    return t;
}

static double dot1_f64(const double* w, const double* x, uint32_t K) {
    v4d a = {0, 0, 0, 0}, b = a, c = a, d = a;
    uint32_t k = 0;
    for (; k + 16 <= K; k += 16) {
        a += ld4(w + k) * ld4(x + k);
        b += ld4(w + k + 4) * ld4(x + k + 4);
        c += ld4(w + k + 8) * ld4(x + k + 8);
        d += ld4(w + k + 12) * ld4(x + k + 12);
    }
    double t = hsum4((a + b) + (c + d));
    for (; k < K; ++k) t += w[k] * x[k];
    return t;
}

/* linear.metal:82-109 (f16 GEMV), 440-474 (int4 GEMV: exact fp32 dequant),
 * 253-343 / 492-574 (GEMMs: int4 dequant rounded to half, linear.metal:538),
 * 113-138 / 347-423 (SiLU epilogue), activations.metal:24-32 (residual add).
 * round_dequant = 1 selects the GEMM rounding of the dequantized weight. */
void orc_linear(const void* x, uint32_t x_stride, const void* w, const void* s, void* y,
                uint32_t y_stride, const void* residual, uint32_t M, uint32_t N, uint32_t K,
                int wfmt, int act, int epi, int round_dequant) {
    if (x_stride == 0) x_stride = K;
    if (y_stride == 0) y_stride = N;
    double* xd = (double*)malloc(sizeof(double) * (size_t)M * K);
    for (uint32_t m = 0; m < M; ++m)
        for (uint32_t k = 0; k < K; ++k) xd[(size_t)m * K + k] = ld(x, (size_t)m * x_stride + k, act);
#pragma omp parallel
    {
        float* wr = (float*)malloc(sizeof(float) * K);
        double* wd = (double*)malloc(sizeof(double) * K);
#pragma omp for schedule(static)
        for (int64_t n = 0; n < (int64_t)N; ++n) {
            deq_row(w, s, wr, (uint32_t)n, K, wfmt, act);
            if (round_dequant && wfmt != LSSM_W_DENSE)
                for (uint32_t k = 0; k < K; ++k) wr[k] = rnd(wr[k], act);
            for (uint32_t k = 0; k < K; ++k) wd[k] = wr[k];
            double dots[4];
            for (uint32_t m = 0; m < M; ++m) {
                if (g_accum_f32) dots[m % 4] = dot1_f32(wd, xd + (size_t)m * K, K);
                else if (m % 4 == 0 && M - m >= 4) dot4_f64(wd, xd + (size_t)m * K, K, dots);
                else if (M - (m - m % 4) < 4) dots[m % 4] = dot1_f64(wd, xd + (size_t)m * K, K);
                float a = (float)dots[m % 4];
                size_t yi = (size_t)m * y_stride + (size_t)n;
                if (epi == LSSM_EPI_SILU) a = silu_f(a);
                if (epi == LSSM_EPI_ADD) a = ld(residual, yi, act) + rnd(a, act);
                st(y, yi, act, a);
            }
        }
        free(wr);
        free(wd);
    }
    free(xd);
}

/* activations.metal:12-21 */
void orc_silu(const void* x, void* y, uint32_t n, int act) {
    for (uint32_t i = 0; i < n; ++i) st(y, i, act, silu_f(ld(x, i, act)));
}

/* activations.metal:24-32 */
void orc_add_inplace(void* y, const void* x, uint32_t n, int act) {
    for (uint32_t i = 0; i < n; ++i) st(y, i, act, ld(y, i, act) + ld(x, i, act));
}

/* activations.metal:76-87 — y = r(silu(x) * gate) */
void orc_silu_gated(const void* x, const void* gate, void* y, uint32_t n, int act) {
    for (uint32_t i = 0; i < n; ++i) st(y, i, act, silu_f(ld(x, i, act)) * ld(gate, i, act));
}

/* activations.metal:49-73 */
void orc_split_silu_xbc(const void* xBC, void* x, void* B, void* C, uint32_t rows,
                        uint32_t d_inner, uint32_t d_state, uint32_t n_groups, int act) {
    uint32_t GN = n_groups * d_state;
    uint32_t dim = d_inner + 2u * GN;
    for (uint32_t t = 0; t < rows; ++t) {
        for (uint32_t f = 0; f < dim; ++f) {
            float v = silu_f(ld(xBC, (size_t)t * dim + f, act));
            if (f < d_inner) st(x, (size_t)t * d_inner + f, act, v);
            else if (f < d_inner + GN) st(B, (size_t)t * GN + (f - d_inner), act, v);
            else st(C, (size_t)t * GN + (f - d_inner - GN), act, v);
        }
    }
}

/* conv1d.metal:63-93 — y[b,t,d] = r(bias[d] + sum_tap w[d,tap] * x[b, t-(K-1-tap), d]) */
void orc_conv1d(const void* x, const void* w, const void* bias, void* y, uint32_t B, uint32_t L,
                uint32_t D, uint32_t K, int act) {
#pragma omp parallel for schedule(static)
    for (int64_t bt = 0; bt < (int64_t)B * L; ++bt) {
        uint32_t b = (uint32_t)(bt / L), t = (uint32_t)(bt % L);
        for (uint32_t d = 0; d < D; ++d) {
            float acc = bias ? ld(bias, d, act) : 0.0f;
            for (uint32_t tap = 0; tap < K; ++tap) {
                int src = (int)t - (int)(K - 1 - tap);
                float v = 0.0f;
                if (src >= 0) v = ld(x, ((size_t)b * L + (uint32_t)src) * D + d, act);
                acc += ld(w, (size_t)d * K + tap, act) * v;
            }
            st(y, ((size_t)b * L + t) * D + d, act, acc);
        }
    }
}

/* conv1d.metal:108-137 — shift the (D,K) window, append x, y = r(bias + sum s*w) */
void orc_conv1d_update(const void* x_new, void* state, const void* w, const void* bias, void* y,
                       uint32_t B, uint32_t D, uint32_t K, int act) {
    for (uint32_t b = 0; b < B; ++b) {
        for (uint32_t d = 0; d < D; ++d) {
            size_t sb = ((size_t)b * D + d) * K;
            for (uint32_t k = 0; k + 1 < K; ++k) st(state, sb + k, act, ld(state, sb + k + 1, act));
            st(state, sb + K - 1, act, ld(x_new, (size_t)b * D + d, act));
            float acc = bias ? ld(bias, d, act) : 0.0f;
            for (uint32_t k = 0; k < K; ++k) acc += ld(state, sb + k, act) * ld(w, (size_t)d * K + k, act);
            st(y, (size_t)b * D + d, act, acc);
        }
    }
}

/* conv1d.metal:35-51 — state[b,d,k] = xBC[b, L-K+k, d] or 0 */
void orc_conv1d_seed(const void* xBC, void* state, uint32_t B, uint32_t L, uint32_t D, uint32_t K,
                     int act) {
    for (uint32_t b = 0; b < B; ++b)
        for (uint32_t d = 0; d < D; ++d)
            for (uint32_t k = 0; k < K; ++k) {
                int src = (int)L - (int)K + (int)k;
                float v = 0.0f;
                if (src >= 0) v = ld(xBC, ((size_t)b * L + (uint32_t)src) * D + d, act);
                st(state, ((size_t)b * D + d) * K + k, act, v);
            }
}

/* activations.metal:76-87 then norm.metal:52-79 over the full row
 * (mamba2_block.cpp:230-238): g = r(silu(z)*y); out = r(g*w*rsqrt(mean g^2+eps)) */
void orc_gated_rmsnorm(const void* z, const void* y, const void* w, void* out, uint32_t rows,
                       uint32_t dim, float eps, int act) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < (int64_t)rows; ++r) {
        size_t base = (size_t)r * dim;
        float* g = (float*)malloc(sizeof(float) * dim);
        double ss = 0.0;
        for (uint32_t i = 0; i < dim; ++i) {
            g[i] = rnd(silu_f(ld(z, base + i, act)) * ld(y, base + i, act), act);
            ss += (double)g[i] * (double)g[i];
        }
        float rrms = 1.0f / sqrtf((float)ss / (float)dim + eps);
        for (uint32_t i = 0; i < dim; ++i) st(out, base + i, act, g[i] * ld(w, i, act) * rrms);
        free(g);
    }
}

/* fused.metal:43-165 — in_proj (dense) + conv1d + SiLU split for L <= 16.
 * The conv reads the UNROUNDED fp32 projection (fused.metal:140-149); z, dt and
 * the pre-conv xBC copy are rounded once. */
void orc_inproj_fused(const void* normed, const void* W_in, const void* W_conv,
                      const void* conv_b, void* proj_z, void* ssd_x, void* ssd_B, void* ssd_C,
                      void* proj_dt, void* proj_xBC, lssm_fused_inproj_dims d, int act) {
    uint32_t L = d.L, K = d.d_model, d_inner = d.d_inner;
    uint32_t GN = d.n_groups * d.d_state;
    uint32_t xBC_dim = d_inner + 2u * GN;
    uint32_t P = d.proj_dim;
    float* acc = (float*)malloc(sizeof(float) * (size_t)L * P);
#pragma omp parallel for schedule(static)
    for (int64_t c = 0; c < (int64_t)P; ++c) {
        for (uint32_t m = 0; m < L; ++m) {
            double a = 0.0;
            for (uint32_t k = 0; k < K; ++k)
                a += (double)ld(normed, (size_t)m * K + k, act) * (double)ld(W_in, (size_t)c * K + k, act);
            acc[(size_t)m * P + c] = (float)a;
        }
    }
    for (uint32_t m = 0; m < L; ++m) {
        for (uint32_t gc = 0; gc < P; ++gc) {
            float v = acc[(size_t)m * P + gc];
            if (gc < d_inner) {
                st(proj_z, (size_t)m * d_inner + gc, act, v);
            } else if (gc < d_inner + xBC_dim) {
                uint32_t c = gc - d_inner;
                st(proj_xBC, (size_t)m * xBC_dim + c, act, v);
                float sum = ld(conv_b, c, act);
                for (uint32_t kk = 0; kk < d.d_conv; ++kk) {
                    int sm = (int)m - (int)(d.d_conv - 1 - kk);
                    if (sm >= 0) sum += ld(W_conv, (size_t)c * d.d_conv + kk, act) * acc[(size_t)sm * P + gc];
                }
                float sv = silu_f(sum);
                if (c < d_inner) st(ssd_x, (size_t)m * d_inner + c, act, sv);
                else if (c < d_inner + GN) st(ssd_B, (size_t)m * GN + (c - d_inner), act, sv);
                else st(ssd_C, (size_t)m * GN + (c - d_inner - GN), act, sv);
            } else {
                st(proj_dt, (size_t)m * d.n_heads + (gc - d_inner - xBC_dim), act, v);
            }
        }
    }
    free(acc);
}

/* ssd_chunked.metal:82-297, per (batch, head), chunks walked in order:
 *   S = r(state)                                   (:124-128)
 *   DT_t = clamp(softplus(dt_raw+dt_bias))          (:138-142)
 *   Lcum = inclusive cumsum(A*DT)                   (:153-187)
 *   M[t,j] = r((C_t.B_j) * e^{Lcum_t-Lcum_j} * DT_j), j<=t      (:204-219)
 *   y[t,p] = r(sum_j M[t,j] X[j,p] + e^{Lcum_t} (C_t.S_p) + D x[t,p]) (:231-263)
 *   S[p,n] = r(e^{L_end} S[p,n] + sum_j e^{L_end-Lcum_j} DT_j B[j,n] X[j,p]) (:275-289)
 *   state = S (fp32 of the rounded value)           (:292-296) */
void orc_ssd_chunked(const void* X, const void* Bp, const void* Cp, const void* dt_raw,
                     const void* dt_bias, const void* A_log, const void* D_skip, void* Y,
                     float* state, uint32_t batch, lssm_ssd_dims d, int act) {
    const uint32_t L = d.L, H = d.H, P = d.P, N = d.N, G = d.n_groups ? d.n_groups : 1;
    const uint32_t CK = d.chunk_size;
    const uint32_t GN = G * N;
    const uint32_t hpg = (H / G) > 0 ? H / G : 1;
#pragma omp parallel for schedule(dynamic)
    for (int64_t bh = 0; bh < (int64_t)batch * H; ++bh) {
        uint32_t b = (uint32_t)(bh / H), h = (uint32_t)(bh % H);
        uint32_t g = h / hpg;
        float A_h = -expf(ld(A_log, h, act));
        float dt_b = ld(dt_bias, h, act);
        float D_h = d.has_D ? ld(D_skip, h, act) : 0.0f;
        float* S = (float*)malloc(sizeof(float) * P * N);
        float* DT = (float*)malloc(sizeof(float) * CK);
        float* Lc = (float*)malloc(sizeof(float) * CK);
        float* M = (float*)malloc(sizeof(float) * CK * CK);
        float* Snew = (float*)malloc(sizeof(float) * P * N);
        float* st_h = state + ((size_t)b * H + h) * P * N;
        for (uint32_t i = 0; i < P * N; ++i) S[i] = rnd(st_h[i], act);
        const size_t xb = (size_t)b * L * H * P, bb = (size_t)b * L * GN, db = (size_t)b * L * H;
        for (uint32_t t0 = 0; t0 < L; t0 += CK) {
            uint32_t tl = (L - t0 < CK) ? L - t0 : CK;
            double run = 0.0;
            for (uint32_t t = 0; t < tl; ++t) {
                float dv = ld(dt_raw, db + (size_t)(t0 + t) * H + h, act) + dt_b;
                DT[t] = clampf_(softplus_f(dv), d.dt_min, d.dt_max);
                run += (double)(A_h * DT[t]);
                Lc[t] = (float)run;
            }
            float L_end = Lc[tl - 1];
            float decay_chunk = expf(L_end);
            for (uint32_t t = 0; t < tl; ++t) {
                for (uint32_t j = 0; j < tl; ++j) {
                    if (j > t) { M[t * CK + j] = 0.0f; continue; }
                    double cb = 0.0;
                    for (uint32_t n = 0; n < N; ++n)
                        cb += (double)ld(Cp, bb + (size_t)(t0 + t) * GN + g * N + n, act) *
                              (double)ld(Bp, bb + (size_t)(t0 + j) * GN + g * N + n, act);
                    float decay = expf(Lc[t] - Lc[j]);
                    M[t * CK + j] = rnd((float)cb * decay * DT[j], act);
                }
            }
            for (uint32_t t = 0; t < tl; ++t) {
                float eLt = expf(Lc[t]);
                for (uint32_t p = 0; p < P; ++p) {
                    double yi = 0.0;
                    for (uint32_t j = 0; j <= t; ++j)
                        yi += (double)M[t * CK + j] * (double)ld(X, xb + (size_t)(t0 + j) * H * P + h * P + p, act);
                    double yo = 0.0;
                    for (uint32_t n = 0; n < N; ++n)
                        yo += (double)ld(Cp, bb + (size_t)(t0 + t) * GN + g * N + n, act) * (double)S[p * N + n];
                    float xc = ld(X, xb + (size_t)(t0 + t) * H * P + h * P + p, act);
                    float yv = (float)yi + (float)yo * eLt + D_h * xc;
                    st(Y, xb + (size_t)(t0 + t) * H * P + h * P + p, act, yv);
                }
            }
            for (uint32_t p = 0; p < P; ++p) {
                for (uint32_t n = 0; n < N; ++n) {
                    double acc = (double)(decay_chunk * S[p * N + n]);
                    for (uint32_t j = 0; j < tl; ++j) {
                        float wj = expf(L_end - Lc[j]) * DT[j];
                        acc += (double)wj * (double)ld(Bp, bb + (size_t)(t0 + j) * GN + g * N + n, act) *
                               (double)ld(X, xb + (size_t)(t0 + j) * H * P + h * P + p, act);
                    }
                    Snew[p * N + n] = rnd((float)acc, act);
                }
            }
            memcpy(S, Snew, sizeof(float) * P * N);
        }
        for (uint32_t i = 0; i < P * N; ++i) st_h[i] = S[i];
        free(S); free(DT); free(Lc); free(M); free(Snew);
    }
}

/* ssd_step.metal:33-77 — s = e^{A dt} s + dt B x (fp32 state); y = r(C.s + D x) */
void orc_ssd_step(const void* x, const void* Bp, const void* Cp, const void* dt_raw,
                  const void* dt_bias, const void* A_log, const void* D_skip, float* state,
                  void* y, uint32_t batch, lssm_ssd_step_dims d, int act) {
    const uint32_t H = d.H, P = d.P, N = d.N, G = d.n_groups ? d.n_groups : 1;
    const uint32_t hpg = (H / G) > 0 ? H / G : 1;
#pragma omp parallel for schedule(static)
    for (int64_t bh = 0; bh < (int64_t)batch * H; ++bh) {
        uint32_t b = (uint32_t)(bh / H), h = (uint32_t)(bh % H);
        uint32_t g = h / hpg;
        float A_h = -expf(ld(A_log, h, act));
        float dt = clampf_(softplus_f(ld(dt_raw, (size_t)b * H + h, act) + ld(dt_bias, h, act)),
                           d.dt_min, d.dt_max);
        float decay = expf(A_h * dt);
        float D_h = d.has_D ? ld(D_skip, h, act) : 0.0f;
        for (uint32_t p = 0; p < P; ++p) {
            float xv = ld(x, ((size_t)b * H + h) * P + p, act);
            float* S = state + (((size_t)b * H + h) * P + p) * N;
            double ys = 0.0;
            for (uint32_t n = 0; n < N; ++n) {
                float bn = ld(Bp, ((size_t)b * G + g) * N + n, act);
                float cn = ld(Cp, ((size_t)b * G + g) * N + n, act);
                float s = decay * S[n] + dt * bn * xv;
                S[n] = s;
                ys += (double)cn * (double)s;
            }
            st(y, ((size_t)b * H + h) * P + p, act, (float)ys + D_h * xv);
        }
    }
}

/* mamba2_model.cpp:128-137 */
void orc_embed(const void* table, const int32_t* ids, void* out, uint32_t n, uint32_t d_model,
               int act) {
    size_t es = esz(act);
    for (uint32_t i = 0; i < n; ++i)
        memcpy((char*)out + (size_t)i * d_model * es, (const char*)table + (size_t)ids[i] * d_model * es,
               (size_t)d_model * es);
}

/* sampler.cpp:13-21 — first index of the maximum (strict > keeps the first) */
void orc_argmax(const void* logits, int32_t* ids, uint32_t rows, uint32_t vocab, int act) {
    for (uint32_t r = 0; r < rows; ++r) {
        size_t base = (size_t)r * vocab;
        uint32_t best = 0;
        float bv = ld(logits, base, act);
        for (uint32_t i = 1; i < vocab; ++i) {
            float v = ld(logits, base + i, act);
            if (v > bv) { bv = v; best = i; }
        }
        ids[r] = (int32_t)best;
    }
}

/* ------------------------------------------------------------------------- */
/* whole model                                                                */
/* ------------------------------------------------------------------------- */
#define RMS_EPS 1e-5f   /* mamba2_block.cpp:45 */
#define DT_MIN 1e-6f    /* mamba2_block.cpp:43 */
#define DT_MAX 1e6f     /* mamba2_block.cpp:44 */

typedef struct {
    uint32_t d_model, d_inner, xbc, proj, H, P, N, G, K, vocab;
} dims_t;

static dims_t dims_of(const lssm_model_config* c) {
    dims_t d;
    d.d_model = c->d_model;
    d.d_inner = c->expand * c->d_model;
    d.G = c->n_groups ? c->n_groups : 1;
    d.N = c->d_state;
    d.xbc = d.d_inner + 2u * d.G * d.N;
    d.H = c->n_heads;
    d.P = c->d_head;
    d.proj = d.d_inner + d.xbc + d.H;
    d.K = c->d_conv;
    d.vocab = c->vocab_size;
    return d;
}

/* Mamba2Model::run_block (mamba2_block.cpp:51-290) for `batch` sequences of
 * `L` rows each (decode: L == 1, conv/ssd step kernels).  hidden [batch*L, d_model]. */
static void run_block(const orc_model* m, uint32_t li, void* hidden, void* conv_state,
                      float* ssd_state, uint32_t batch, uint32_t L, int decode) {
    const lssm_model_config* c = &m->cfg;
    const lssm_layer_weights* bw = &m->layers[li];
    dims_t d = dims_of(c);
    int act = (int)c->act, wf = (int)c->wfmt;
    size_t es = esz(act);
    size_t R = (size_t)batch * L;
    void* normed = malloc(R * d.d_model * es);
    void* proj = malloc(R * d.proj * es);
    void* z = malloc(R * d.d_inner * es);
    void* xbc = malloc(R * d.xbc * es);
    void* dtr = malloc(R * d.H * es);
    void* conv = malloc(R * d.xbc * es);
    void* xs = malloc(R * d.d_inner * es);
    void* Bs = malloc(R * d.G * d.N * es);
    void* Cs = malloc(R * d.G * d.N * es);
    void* ys = malloc(R * d.d_inner * es);
    void* gn = malloc(R * d.d_inner * es);
    void* out = malloc(R * d.d_model * es);

    orc_rmsnorm(hidden, bw->norm_w, normed, (uint32_t)R, d.d_model, RMS_EPS, act);
    char* cs = (char*)conv_state + (size_t)li * batch * d.xbc * d.K * es;
    float* ss = ssd_state + (size_t)li * batch * d.H * d.P * d.N;
    /* mamba2_block.cpp:97-98,130-148: a short prefill (1 < L <= 16) of fp16
     * weights runs the fused in_proj + conv + SiLU split, whose conv reads the
     * unrounded fp32 projection (fused.metal:137-149); per sequence, as the
     * reference's batch-1 model does. */
    const int fused = !decode && L > 1 && L <= 16 && wf == LSSM_W_DENSE && act == LSSM_F16;
    int rd = !(decode || L == 1);
    const int step = decode || L == 1;
    if (fused) {
        size_t GN = (size_t)d.G * d.N;
        lssm_fused_inproj_dims fd = {L, d.d_model, d.d_inner, d.N, d.G, d.H, d.K, d.proj};
        for (uint32_t b = 0; b < batch; ++b) {
            size_t r0 = (size_t)b * L;
            orc_inproj_fused((char*)normed + r0 * d.d_model * es, bw->in_proj_w, bw->conv1d_w,
                             bw->conv1d_b, (char*)z + r0 * d.d_inner * es, (char*)xs + r0 * d.d_inner * es,
                             (char*)Bs + r0 * GN * es, (char*)Cs + r0 * GN * es, (char*)dtr + r0 * d.H * es,
                             (char*)xbc + r0 * d.xbc * es, fd, act);
        }
    } else {
        /* three in_proj slices (mamba2_block.cpp:150-152): same math as one
         * projection over all rows; GEMV semantics for decode / L == 1. */
        orc_linear(normed, 0, bw->in_proj_w, bw->in_proj_s, proj, 0, NULL, (uint32_t)R, d.proj,
                   d.d_model, wf, act, LSSM_EPI_NONE, rd);
        for (size_t r = 0; r < R; ++r) {
            memcpy((char*)z + r * d.d_inner * es, (char*)proj + r * d.proj * es, d.d_inner * es);
            memcpy((char*)xbc + r * d.xbc * es, (char*)proj + (r * d.proj + d.d_inner) * es, d.xbc * es);
            memcpy((char*)dtr + r * d.H * es, (char*)proj + (r * d.proj + d.d_inner + d.xbc) * es, d.H * es);
        }
        /* mamba2_block.cpp:155-170, 183-217: one-row passes (decode, or a 1-token
         * prefill) use the conv update and the SSD step kernels. */
        if (step) {
            orc_conv1d_update(xbc, cs, bw->conv1d_w, bw->conv1d_b, conv, batch, d.xbc, d.K, act);
        } else {
            orc_conv1d(xbc, bw->conv1d_w, bw->conv1d_b, conv, batch, L, d.xbc, d.K, act);
        }
        orc_split_silu_xbc(conv, xs, Bs, Cs, (uint32_t)R, d.d_inner, d.N, d.G, act);
    }
    if (step) {
        lssm_ssd_step_dims sd = {d.H, d.P, d.N, d.G, DT_MIN, DT_MAX, 1u};
        orc_ssd_step(xs, Bs, Cs, dtr, bw->dt_bias, bw->A_log, bw->D, ss, ys, batch, sd, act);
    } else {
        uint32_t ck = c->chunk_size;
        if (ck > L) ck = L;
        if (ck > 64) ck = 64;                       /* mamba2_block.cpp:203-206 */
        lssm_ssd_dims sd = {L, d.H, d.P, d.N, d.G, ck, DT_MIN, DT_MAX, 1u};
        orc_ssd_chunked(xs, Bs, Cs, dtr, bw->dt_bias, bw->A_log, bw->D, ys, ss, batch, sd, act);
    }
    orc_gated_rmsnorm(z, ys, bw->mixer_norm_w, gn, (uint32_t)R, d.d_inner, RMS_EPS, act);
    orc_linear(gn, 0, bw->out_proj_w, bw->out_proj_s, out, 0, NULL, (uint32_t)R, d.d_model,
               d.d_inner, wf, act, LSSM_EPI_NONE, rd);
    orc_add_inplace(hidden, out, (uint32_t)(R * d.d_model), act);
    if (!decode) orc_conv1d_seed(xbc, cs, batch, L, d.xbc, d.K, act);

    free(normed); free(proj); free(z); free(xbc); free(dtr); free(conv);
    free(xs); free(Bs); free(Cs); free(ys); free(gn); free(out);
}

/* run_block for one layer on caller-provided hidden rows (the layer-by-layer
 * parity checks feed it the GPU's hidden state entering layer li). */
void orc_model_block(const orc_model* m, uint32_t li, void* hidden, void* conv_state, float* ssd_state,
                     uint32_t batch, uint32_t L, int decode) {
    run_block(m, li, hidden, conv_state, ssd_state, batch, L, decode);
}

/* Mamba2Model::compute_logits (mamba2_model.cpp:144-175) for `rows` rows. */
void orc_model_logits(const orc_model* m, const void* rows_h, uint32_t rows, void* logits) {
    const lssm_model_config* c = &m->cfg;
    int act = (int)c->act;
    size_t es = esz(act);
    void* nf = malloc((size_t)rows * c->d_model * es);
    orc_rmsnorm(rows_h, m->norm_f, nf, rows, c->d_model, RMS_EPS, act);
    orc_linear(nf, 0, m->lm_head, NULL, logits, 0, NULL, rows, c->vocab_size, c->d_model,
               LSSM_W_DENSE, act, LSSM_EPI_NONE, 0);
    free(nf);
}

void orc_model_prefill(const orc_model* m, void* conv_state, float* ssd_state, const int32_t* ids,
                       uint32_t batch, uint32_t L, void* logits) {
    const lssm_model_config* c = &m->cfg;
    int act = (int)c->act;
    size_t es = esz(act);
    size_t R = (size_t)batch * L;
    void* hidden = malloc(R * c->d_model * es);
    orc_embed(m->embed, ids, hidden, (uint32_t)R, c->d_model, act);
    for (uint32_t li = 0; li < c->n_layer; ++li)
        run_block(m, li, hidden, conv_state, ssd_state, batch, L, 0);
    void* last = malloc((size_t)batch * c->d_model * es);
    for (uint32_t b = 0; b < batch; ++b)
        memcpy((char*)last + (size_t)b * c->d_model * es,
               (char*)hidden + (((size_t)b * L) + L - 1) * c->d_model * es, c->d_model * es);
    orc_model_logits(m, last, batch, logits);
    free(last);
    free(hidden);
}

void orc_model_decode(const orc_model* m, void* conv_state, float* ssd_state, const int32_t* ids,
                      uint32_t batch, void* logits) {
    const lssm_model_config* c = &m->cfg;
    int act = (int)c->act;
    size_t es = esz(act);
    void* hidden = malloc((size_t)batch * c->d_model * es);
    orc_embed(m->embed, ids, hidden, batch, c->d_model, act);
    for (uint32_t li = 0; li < c->n_layer; ++li)
        run_block(m, li, hidden, conv_state, ssd_state, batch, 1, 1);
    orc_model_logits(m, hidden, batch, logits);
    free(hidden);
}

/*
 * gemm_ref.c — CPU restatement of the skinny decode GEMM and its SwiGLU
 * epilogue.  TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it, as a checker; the product path
 * (libkrk_gemm.so) never does.
 *
 * Reference algorithm restated here (willzeng274/kernel-rush-kawk):
 *   - projection  C = A·Wᵀ, fp32 accumulation, one bf16 rounding at the end:
 *       engine/kernels/gemm.py:54-93 (_skinny_kernel, tl.dot fp32 acc ->
 *       .to(bfloat16) at :90), gemm.py:200-245 (_gemv_kernel: fp32 FMA and
 *       tl.sum, bf16 store at :240); the incumbent is torch `a @ w.t()`
 *       (gemm.py:428), which on CPU is fp32-accumulated bf16 GEMM.
 *   - SwiGLU epilogue with three bf16 roundings:
 *       engine/kernels/gemm.py:107-113 (_swiglu_epilogue),
 *       engine/kernels/swiglu.py:14-24 (gate-first [M, 2I] layout).
 *   - residual add + RMSNorm prologue: xout = bf16(x + y),
 *       n = bf16(bf16(xout·rsqrt(mean(xout²) + eps))·w_norm):
 *       engine/kernels/add_rmsnorm.py:15-29, engine/kernels/gemm.py:21-51,
 *       cast placement engine/kernels/rmsnorm.py:34-43.
 *   - token selection: first index of the maximum
 *       (engine/engine.py:196 `argmax`, OPTIMIZATION_GUIDE.md:213 lowest index).
 *
 * Every function works on raw bf16 bit patterns (uint16_t).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static float bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

/* fp32 -> bf16, round to nearest even; NaN keeps a quiet NaN. */
static uint16_t f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

/* fp64 -> bf16 with a single rounding (round to nearest even).  Going through
 * fp32 first can double-round when the fp32 value lands exactly on a bf16
 * midpoint; that case is steered by the sign of the discarded remainder. */
static uint16_t f64_to_bf16(double d) {
    float f = (float)d;
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    if ((u & 0xffffu) == 0x8000u && (double)f != d) {
        const int above = fabs(d) > fabs((double)f);
        u = above ? u + 1u : u - 1u;
    }
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

/* y[m][n] = bf16( sum_{k=0}^{K-1} x[m][k]·w[n][k] ), fp32 accumulator, k ascending.
 * Strides in elements.  This is the _gemv_kernel / tl.dot contract with one
 * fixed summation order (any order is a valid fp32 reordering). */
void oracle_linear_f32(const uint16_t* x, int64_t ldx, const uint16_t* w, int64_t ldw,
                       uint16_t* y, int64_t ldy, int M, int N, int K) {
    for (int m = 0; m < M; ++m) {
        const uint16_t* xr = x + (int64_t)m * ldx;
        for (int n = 0; n < N; ++n) {
            const uint16_t* wr = w + (int64_t)n * ldw;
            float acc = 0.0f;
            for (int k = 0; k < K; ++k) acc += bf16_to_f32(xr[k]) * bf16_to_f32(wr[k]);
            y[(int64_t)m * ldy + n] = f32_to_bf16(acc);
        }
    }
}

/* Exact reference: fp64 sums (each bf16·bf16 product is exact in fp64), the
 * sum of |products| for error bounds, and the singly-rounded bf16 result.
 * Any of the three outputs may be NULL. */
void oracle_linear_f64(const uint16_t* x, int64_t ldx, const uint16_t* w, int64_t ldw,
                       double* exact, double* abssum, uint16_t* y, int M, int N, int K) {
    for (int m = 0; m < M; ++m) {
        const uint16_t* xr = x + (int64_t)m * ldx;
        for (int n = 0; n < N; ++n) {
            const uint16_t* wr = w + (int64_t)n * ldw;
            double acc = 0.0, mag = 0.0;
            for (int k = 0; k < K; ++k) {
                const double p = (double)bf16_to_f32(xr[k]) * (double)bf16_to_f32(wr[k]);
                acc += p;
                mag += fabs(p);
            }
            const int64_t o = (int64_t)m * N + n;
            if (exact) exact[o] = acc;
            if (abssum) abssum[o] = mag;
            if (y) y[o] = f64_to_bf16(acc);
        }
    }
}

/* out = bf16( bf16(silu_f32(bf16 g)) · bf16 u ) for already-bf16 g and u. */
uint16_t oracle_silu_mul1(uint16_t g, uint16_t u) {
    const float gf = bf16_to_f32(g);
    const float uf = bf16_to_f32(u);
    const float s = bf16_to_f32(f32_to_bf16(gf / (1.0f + expf(-gf))));
    return f32_to_bf16(s * uf);
}

/* SwiGLU over a gate-first [M, 2I] bf16 matrix (engine/kernels/swiglu.py:14-24). */
void oracle_swiglu(const uint16_t* gu, int64_t ldgu, uint16_t* out, int64_t ldo, int M, int I) {
    for (int m = 0; m < M; ++m)
        for (int i = 0; i < I; ++i)
            out[(int64_t)m * ldo + i] = oracle_silu_mul1(gu[(int64_t)m * ldgu + i], gu[(int64_t)m * ldgu + I + i]);
}

/* Fused gate/up: out[m][i] = silu_mul(bf16(x·Wg[i]), bf16(x·Wu[i])), fp32
 * accumulation in k order; w is [2I, K], gate rows first. */
void oracle_gateup_f32(const uint16_t* x, int64_t ldx, const uint16_t* w, int64_t ldw,
                       uint16_t* out, int64_t ldo, int M, int I, int K) {
    for (int m = 0; m < M; ++m) {
        const uint16_t* xr = x + (int64_t)m * ldx;
        for (int i = 0; i < I; ++i) {
            const uint16_t* wg = w + (int64_t)i * ldw;
            const uint16_t* wu = w + (int64_t)(I + i) * ldw;
            float g = 0.0f, u = 0.0f;
            for (int k = 0; k < K; ++k) {
                const float xv = bf16_to_f32(xr[k]);
                g += xv * bf16_to_f32(wg[k]);
                u += xv * bf16_to_f32(wu[k]);
            }
            out[(int64_t)m * ldo + i] = oracle_silu_mul1(f32_to_bf16(g), f32_to_bf16(u));
        }
    }
}

/* First index of the largest value in each row (NaN-free input). */
void oracle_argmax_rows(const uint16_t* v, int64_t ld, int M, int N, int64_t* idx) {
    for (int m = 0; m < M; ++m) {
        const uint16_t* r = v + (int64_t)m * ld;
        int64_t best = 0;
        float bv = bf16_to_f32(r[0]);
        for (int n = 1; n < N; ++n) {
            const float f = bf16_to_f32(r[n]);
            if (f > bv) { bv = f; best = n; }
        }
        idx[m] = best;
    }
}

/* Residual add + RMSNorm over rows of K: xout = bf16(x + y); the mean of
 * squares of xout is taken in fp64 (any fp32 order lies within a few ulp of
 * it) and rstd = 1/sqrt(mean + eps) is rounded to fp32, the precision the
 * reference computes it in; n = bf16(bf16(xout·rstd)·w_norm) with both
 * products in fp32.  rstd_out receives the fp64 value for error analysis. */
void oracle_add_rms_norm(const uint16_t* x, int64_t ldx, const uint16_t* y, int64_t ldy,
                         const uint16_t* w_norm, double eps, uint16_t* xout, uint16_t* n, int64_t ldo,
                         int M, int K, double* rstd_out) {
    for (int m = 0; m < M; ++m) {
        double ss = 0.0;
        for (int k = 0; k < K; ++k) {
            const uint16_t s = f32_to_bf16(bf16_to_f32(x[m * ldx + k]) + bf16_to_f32(y[m * ldy + k]));
            xout[m * ldo + k] = s;
            const double sf = bf16_to_f32(s);
            ss += sf * sf;
        }
        const double rstd = 1.0 / sqrt(ss / K + eps);
        rstd_out[m] = rstd;
        const float r32 = (float)rstd;
        for (int k = 0; k < K; ++k) {
            const float a = bf16_to_f32(f32_to_bf16(bf16_to_f32(xout[m * ldo + k]) * r32));
            n[m * ldo + k] = f32_to_bf16(a * bf16_to_f32(w_norm[k]));
        }
    }
}

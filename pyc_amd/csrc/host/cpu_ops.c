/* cpu_ops.c — fp32 host implementations of the ops the engine's CPU executor
 * runs beyond the reference's F32 MATMUL/ADD/RELU (reference
 * src/compiler/compiler_api.c:1877-2092 fails on every other kind and dtype).
 *
 * They make the CPU executor, which pyc_cuda_dispatch falls back to
 * (reference src/compiler/runtime/cuda_backend.c:2883-2908), total over the
 * modules the GPU backend lowers: bf16/f16 values (decoded to fp32, every op
 * result rounded back to its value's type, as the device stores it), the
 * weight-only fp8 MATMUL, NHWC CONV2D, ATTENTION, GELU and LAYERNORM.
 * Arithmetic is plain fp32 in a fixed order (no FMA contraction is relied
 * on); work is split over PYC_NUM_THREADS threads (default 1, at most 32),
 * the reference executor's threading knob (compiler_api.c:1790-1812).
 *
 * Semantics (the same the device kernels implement):
 *   conv2d     y[n,p,q,k] = sum_{r,s,c} x[n, p*sh-ph+r, q*sw-pw+s, c] w[k,r,s,c],
 *              x NHWC, w KRSC, y NPQK, out-of-image taps zero;
 *   attention  O = softmax(Q K^T * scale (+ causal mask j <= i)) V per (b,h),
 *              [B,H,S,D], max-subtracted, fp32;
 *   fp8 layer  Y[m,n] = scale[n] * sum_k X[m,k] e4m3(Wq[n,k]), Wq stored [N,K];
 *   gelu       0.5 x (1 + erf(x / sqrt 2));
 *   layernorm  (x - mean) / sqrt(var + eps) * gamma + beta over the last dim,
 *              population variance. */
#include "cpu_ops.h"

#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- number formats */

float pyc_cpu_bf16_to_f32(uint16_t h) {
    const uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, sizeof(f));
    return f;
}

uint16_t pyc_cpu_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, sizeof(u));
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu) != 0u) {
        return (uint16_t)((u >> 16) | 0x0040u); /* NaN stays a quiet NaN */
    }
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16); /* nearest, ties to even */
}

float pyc_cpu_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t man = h & 0x3ffu;
    float f;
    uint32_t u;
    if (e == 0x1fu) {
        u = sign | 0x7f800000u | (man << 13);
    } else if (e == 0) {
        /* zero or subnormal: man * 2^-24 is exact in fp32 */
        f = ldexpf((float)man, -24);
        return sign ? -f : f;
    } else {
        u = sign | ((e + 112u) << 23) | (man << 13);
    }
    memcpy(&f, &u, sizeof(f));
    return f;
}

uint16_t pyc_cpu_f32_to_f16(float f) {
    uint32_t u;
    uint16_t sign;
    uint32_t a;
    memcpy(&u, &f, sizeof(u));
    sign = (uint16_t)((u >> 16) & 0x8000u);
    a = u & 0x7fffffffu;
    if (a > 0x7f800000u) {
        return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu)); /* NaN */
    }
    if (a >= 0x477ff000u) {
        return (uint16_t)(sign | 0x7c00u); /* rounds past 65504: inf */
    }
    if (a < 0x38800000u) {
        /* below the smallest normal half (2^-14): the result is a multiple of
         * 2^-24; scaling by 2^24 is exact, nearbyintf rounds ties to even in
         * the default mode, and 1024 comes out as the smallest normal */
        float af;
        float q;
        memcpy(&af, &a, sizeof(af));
        q = nearbyintf(af * 16777216.0f);
        return (uint16_t)(sign | (uint16_t)q);
    }
    {
        /* normal: drop 13 mantissa bits with round to nearest even */
        const uint32_t rounded = a + 0xfffu + ((a >> 13) & 1u);
        return (uint16_t)(sign | (uint16_t)((rounded >> 13) - (112u << 10)));
    }
}

float pyc_cpu_e4m3_to_f32(uint8_t v) {
    /* OCP FP8 E4M3 (e4m3fn): bias 7, no infinities, 0x7f / 0xff are NaN */
    const int sign = v >> 7;
    const int e = (v >> 3) & 0xf;
    const int m = v & 0x7;
    float f;
    if (e == 0xf && m == 0x7) {
        return NAN;
    }
    f = e == 0 ? ldexpf((float)m, -9) : ldexpf((float)(8 + m), e - 10);
    return sign ? -f : f;
}

float pyc_cpu_round_to(pyc_dtype t, float f) {
    if (t == PYC_DTYPE_BF16) {
        return pyc_cpu_bf16_to_f32(pyc_cpu_f32_to_bf16(f));
    }
    if (t == PYC_DTYPE_F16) {
        return pyc_cpu_f16_to_f32(pyc_cpu_f32_to_f16(f));
    }
    return f;
}

/* ---------------------------------------------------------------- op attributes */

void pyc_op_conv_attrs(const char* name, int* sh, int* sw, int* ph, int* pw) {
    const char* at = name ? strchr(name, '@') : NULL;
    *sh = *sw = 1;
    *ph = *pw = 0;
    if (at) {
        int a, b, c, d;
        if (sscanf(at, "@s%dx%dp%dx%d", &a, &b, &c, &d) == 4) {
            *sh = a;
            *sw = b;
            *ph = c;
            *pw = d;
        }
    }
}

int pyc_op_is_causal(const char* name) {
    return name && strstr(name, "causal") != NULL;
}

float pyc_op_eps(const char* name) {
    const char* e = name ? strstr(name, "@eps") : NULL;
    return e ? strtof(e + 4, NULL) : 1e-5f;
}

/* ---------------------------------------------------------------- threading */

int pyc_cpu_threads(size_t work_items) {
    const char* env = getenv("PYC_NUM_THREADS");
    long want = env && env[0] ? strtol(env, NULL, 10) : 1;
    if (want < 1) want = 1;
    if (want > 32) want = 32;
    if ((size_t)want > work_items) want = (long)(work_items ? work_items : 1);
    return (int)want;
}

typedef struct {
    void (*fn)(void*, size_t, size_t);
    void* ctx;
    size_t lo, hi;
} range_job;

static void* range_worker(void* p) {
    range_job* j = (range_job*)p;
    j->fn(j->ctx, j->lo, j->hi);
    return NULL;
}

/* fn(ctx, lo, hi) over [0, n) cut into contiguous ranges, one per thread. */
static void parallel_for(size_t n, void (*fn)(void*, size_t, size_t), void* ctx) {
    const int nt = pyc_cpu_threads(n);
    pthread_t tid[32];
    range_job jobs[32];
    int started[32];
    size_t per, t;
    if (nt <= 1) {
        fn(ctx, 0, n);
        return;
    }
    per = (n + (size_t)nt - 1) / (size_t)nt;
    for (t = 0; t < (size_t)nt; ++t) {
        jobs[t].fn = fn;
        jobs[t].ctx = ctx;
        jobs[t].lo = t * per < n ? t * per : n;
        jobs[t].hi = (t + 1) * per < n ? (t + 1) * per : n;
        started[t] = pthread_create(&tid[t], NULL, range_worker, &jobs[t]) == 0;
        if (!started[t]) {
            fn(ctx, jobs[t].lo, jobs[t].hi);
        }
    }
    for (t = 0; t < (size_t)nt; ++t) {
        if (started[t]) {
            pthread_join(tid[t], NULL);
        }
    }
}

/* ---------------------------------------------------------------- conv2d */

typedef struct {
    const float* x;
    const float* w;
    float* y;
    int N, H, W, C, K, R, S, ph, pw, sh, sw, P, Q;
} conv_ctx;

/* output rows (n, p) in [lo, hi) */
static void conv_rows(void* p, size_t lo, size_t hi) {
    const conv_ctx* c = (const conv_ctx*)p;
    size_t row;
    for (row = lo; row < hi; ++row) {
        const int n = (int)(row / (size_t)c->P);
        const int pp = (int)(row % (size_t)c->P);
        int q, k, r, s, ch;
        for (q = 0; q < c->Q; ++q) {
            float* yo = c->y + (((size_t)n * c->P + pp) * c->Q + q) * c->K;
            for (k = 0; k < c->K; ++k) {
                float acc = 0.0f;
                for (r = 0; r < c->R; ++r) {
                    const int ih = pp * c->sh - c->ph + r;
                    if (ih < 0 || ih >= c->H) continue;
                    for (s = 0; s < c->S; ++s) {
                        const int iw = q * c->sw - c->pw + s;
                        const float* xi;
                        const float* wi;
                        if (iw < 0 || iw >= c->W) continue;
                        xi = c->x + (((size_t)n * c->H + ih) * c->W + iw) * c->C;
                        wi = c->w + (((size_t)k * c->R + r) * c->S + s) * c->C;
                        for (ch = 0; ch < c->C; ++ch) {
                            const float prod = xi[ch] * wi[ch];
                            acc += prod;
                        }
                    }
                }
                yo[k] = acc;
            }
        }
    }
}

void pyc_cpu_conv2d_nhwc(const float* x, const float* w, float* y, int N, int H, int W, int C, int K, int R, int S,
                         int ph, int pw, int sh, int sw) {
    conv_ctx c;
    c.x = x;
    c.w = w;
    c.y = y;
    c.N = N;
    c.H = H;
    c.W = W;
    c.C = C;
    c.K = K;
    c.R = R;
    c.S = S;
    c.ph = ph;
    c.pw = pw;
    c.sh = sh;
    c.sw = sw;
    c.P = (H + 2 * ph - R) / sh + 1;
    c.Q = (W + 2 * pw - S) / sw + 1;
    parallel_for((size_t)N * c.P, conv_rows, &c);
}

/* ---------------------------------------------------------------- attention */

typedef struct {
    const float* q;
    const float* k;
    const float* v;
    float* o;
    int S, D, causal;
    float scale;
    float* rows;    /* one score row of S floats per thread's range */
    size_t per;     /* heads per range (the range of head lo is lo / per) */
} attn_ctx;

static void attn_heads(void* p, size_t lo, size_t hi) {
    const attn_ctx* a = (const attn_ctx*)p;
    const int S = a->S, D = a->D;
    float* sc = a->rows + (lo / a->per) * (size_t)S;
    size_t bh;
    for (bh = lo; bh < hi; ++bh) {
        const float* qb = a->q + bh * (size_t)S * D;
        const float* kb = a->k + bh * (size_t)S * D;
        const float* vb = a->v + bh * (size_t)S * D;
        float* ob = a->o + bh * (size_t)S * D;
        int i, j, d;
        for (i = 0; i < S; ++i) {
            const int jend = a->causal ? i + 1 : S;
            float mx = -INFINITY;
            float denom = 0.0f;
            for (j = 0; j < jend; ++j) {
                float dot = 0.0f;
                for (d = 0; d < D; ++d) {
                    const float prod = qb[(size_t)i * D + d] * kb[(size_t)j * D + d];
                    dot += prod;
                }
                sc[j] = dot * a->scale;
                if (sc[j] > mx) mx = sc[j];
            }
            for (j = 0; j < jend; ++j) {
                sc[j] = expf(sc[j] - mx);
                denom += sc[j];
            }
            for (d = 0; d < D; ++d) {
                float acc = 0.0f;
                for (j = 0; j < jend; ++j) {
                    const float prod = sc[j] * vb[(size_t)j * D + d];
                    acc += prod;
                }
                ob[(size_t)i * D + d] = acc / denom;
            }
        }
    }
}

int pyc_cpu_attention(const float* q, const float* k, const float* v, float* o, int B, int H, int S, int D,
                      int causal, float scale) {
    const size_t heads = (size_t)B * H;
    const int nt = pyc_cpu_threads(heads);
    attn_ctx a;
    a.q = q;
    a.k = k;
    a.v = v;
    a.o = o;
    a.S = S;
    a.D = D;
    a.causal = causal;
    a.scale = scale;
    if (heads == 0) {
        return 0;
    }
    /* the ranges parallel_for cuts: ceil(heads / nt) heads each */
    a.per = nt <= 1 ? heads : (heads + (size_t)nt - 1) / (size_t)nt;
    a.rows = (float*)malloc((size_t)(nt > 1 ? nt : 1) * (size_t)S * sizeof(float));
    if (!a.rows) {
        return -1;
    }
    parallel_for(heads, attn_heads, &a);
    free(a.rows);
    return 0;
}

/* ---------------------------------------------------------------- fp8-weight GEMM */

typedef struct {
    const float* x;
    const uint8_t* wq;
    const float* scale;
    float* y;
    const float* lut;
    int M, N, K;
} w8_ctx;

static void w8_cols(void* p, size_t lo, size_t hi) {
    const w8_ctx* c = (const w8_ctx*)p;
    size_t n;
    int m, kk;
    for (n = lo; n < hi; ++n) {
        const uint8_t* wr = c->wq + n * (size_t)c->K;
        for (m = 0; m < c->M; ++m) {
            const float* xr = c->x + (size_t)m * c->K;
            float acc = 0.0f;
            for (kk = 0; kk < c->K; ++kk) {
                const float prod = xr[kk] * c->lut[wr[kk]];
                acc += prod;
            }
            c->y[(size_t)m * c->N + n] = acc * c->scale[n];
        }
    }
}

void pyc_cpu_w8a16_gemm(const float* x, const uint8_t* wq, const float* scale, float* y, int M, int N, int K) {
    float lut[256];
    w8_ctx c;
    int i;
    for (i = 0; i < 256; ++i) lut[i] = pyc_cpu_e4m3_to_f32((uint8_t)i);
    c.x = x;
    c.wq = wq;
    c.scale = scale;
    c.y = y;
    c.lut = lut;
    c.M = M;
    c.N = N;
    c.K = K;
    parallel_for((size_t)N, w8_cols, &c);
}

/* ---------------------------------------------------------------- GELU / LayerNorm */

void pyc_cpu_gelu(const float* x, float* y, size_t n) {
    size_t i;
    for (i = 0; i < n; ++i) {
        const double v = (double)x[i];
        y[i] = (float)(0.5 * v * (1.0 + erf(v * 0.70710678118654752440)));
    }
}

void pyc_cpu_layernorm(const float* x, const float* gamma, const float* beta, float* y, size_t rows, size_t D,
                       float eps) {
    size_t r, j;
    for (r = 0; r < rows; ++r) {
        const float* xr = x + r * D;
        float* yr = y + r * D;
        double mean = 0.0, var = 0.0, inv;
        for (j = 0; j < D; ++j) mean += (double)xr[j];
        mean /= (double)D;
        for (j = 0; j < D; ++j) {
            const double d = (double)xr[j] - mean;
            var += d * d;
        }
        var /= (double)D;
        inv = 1.0 / sqrt(var + (double)eps);
        for (j = 0; j < D; ++j) {
            double v = ((double)xr[j] - mean) * inv;
            if (gamma) v *= (double)gamma[j];
            if (beta) v += (double)beta[j];
            yr[j] = (float)v;
        }
    }
}

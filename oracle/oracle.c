/* oracle.c — CPU restatement of PyC's CPU executor and fp32 reference ops.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker for the HIP backend: it
 * is compiled into oracle/_build/liboracle.so and loaded by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg, never by the
 * product library (pyc_amd/), which fails loudly without its HIP build.
 *
 * Functions and what pins each (the tests that pin them live in
 * tests/test_oracle.py):
 *   orc_matmul_f32        reference compiler_api.c:1747-1875 (matmul_compute_rows /
 *                         matmul_tiled_f32): k ascending in blocks of 64, fp32
 *                         multiply then add per step, row split over threads.
 *                         Pinned: KAT test_cpu_execution.c:56-59, bit-equality with
 *                         oracle/_ref (the reference engine itself), fp64 numpy.
 *   orc_add_epilogue      reference cuda_backend.c:1697-1731 (MATRIX / ROW_BIAS /
 *                         SCALAR add modes), orc_relu: cuda_backend.c:1733-1742.
 *                         Pinned: KAT test_cuda_backend.c:84-89 and oracle/_ref
 *                         run with PYC_CUDA_SIMULATE_AVAILABLE.
 *   orc_f32_to_bf16 / orc_bf16_to_f32
 *                         round-to-nearest-even as reference
 *                         benchmark/.../pyc_compiler_next_bench.c:248-256, plus NaN
 *                         kept quiet. Pinned: torch.bfloat16 conversion.
 *   orc_e4m3_to_f32 / orc_f32_to_e4m3
 *                         OCP FP8 E4M3 (e4m3fn: bias 7, no inf, 0x7F/0xFF NaN,
 *                         max 448), RNE with saturation. No reference counterpart
 *                         (the reference has no fp8). Pinned: torch.float8_e4m3fn,
 *                         exhaustively over all 256 codes.
 *   orc_gemm_bf16         fp32 CPU GEMM on exactly decoded bf16 inputs, same
 *                         accumulation order as orc_matmul_f32; rows [r0,r1).
 *   orc_attention_f32     softmax(QK^T*scale + causal mask) V per (b,h), fp32,
 *                         max-subtracted. No reference counterpart (the reference
 *                         kernel is an identity copy, attention/kernel.cu:30-59).
 *                         Pinned: torch scaled_dot_product_attention in fp64 and
 *                         the invariants row0==V[0], constant V, scale 0 => prefix mean.
 *   orc_conv2d_nhwc_f32   direct NHWC/KRSC cross-correlation + bias + relu, the
 *                         semantics of reference conv2d/kernel.cu:24-44 (CUTLASS
 *                         fprop, not buildable here). Pinned: scipy.signal.correlate,
 *                         1x1 filter == GEMM, delta filter == shift.
 *   orc_w8a16_layer       Y = relu?((X * dequant(Wq)^T) * scale[n]) rounded to bf16.
 *                         Pinned: fp64 numpy on torch-decoded e4m3 weights.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- bf16 */

uint16_t orc_f32_to_bf16(float f) {
    uint32_t bits;
    memcpy(&bits, &f, sizeof(bits));
    if ((bits & 0x7f800000u) == 0x7f800000u && (bits & 0x007fffffu) != 0u) {
        /* NaN: keep sign, force a quiet payload bit so truncation stays NaN. */
        return (uint16_t)((bits >> 16) | 0x0040u);
    }
    {
        uint32_t lsb = (bits >> 16) & 1u;
        uint32_t rounded = bits + 0x7fffu + lsb;
        return (uint16_t)(rounded >> 16);
    }
}

float orc_bf16_to_f32(uint16_t h) {
    uint32_t bits = ((uint32_t)h) << 16;
    float f;
    memcpy(&f, &bits, sizeof(f));
    return f;
}

void orc_f32_to_bf16_array(const float* in, uint16_t* out, size_t n) {
    size_t i;
    for (i = 0; i < n; ++i) {
        out[i] = orc_f32_to_bf16(in[i]);
    }
}

void orc_bf16_to_f32_array(const uint16_t* in, float* out, size_t n) {
    size_t i;
    for (i = 0; i < n; ++i) {
        out[i] = orc_bf16_to_f32(in[i]);
    }
}

/* ---------------------------------------------------------------- fp8 e4m3fn */

float orc_e4m3_to_f32(uint8_t v) {
    int sign = (v >> 7) & 1;
    int exp = (v >> 3) & 0xf;
    int man = v & 0x7;
    float mag;
    if (exp == 0xf && man == 0x7) {
        return NAN;
    }
    if (exp == 0) {
        mag = ldexpf((float)man, -9); /* subnormal: man/8 * 2^-6 */
    } else {
        mag = ldexpf((float)(8 + man), exp - 10); /* (1+man/8) * 2^(exp-7) */
    }
    return sign ? -mag : mag;
}

/* Round-to-nearest-even onto the e4m3fn grid, saturating to +-448 (the
 * "satfinite" convention of fp8 weight quantizers). NaN maps to 0x7F. */
uint8_t orc_f32_to_e4m3(float f) {
    uint8_t sign;
    float a;
    int e;
    float q;
    int code;
    if (isnan(f)) {
        return 0x7f;
    }
    sign = (uint8_t)(signbit(f) ? 0x80 : 0x00);
    a = fabsf(f);
    if (a >= 448.0f) {
        return (uint8_t)(sign | 0x7e);
    }
    if (a < ldexpf(1.0f, -6)) {
        /* subnormal grid: multiples of 2^-9 */
        q = nearbyintf(a * 512.0f); /* default rounding mode: to nearest even */
        code = (int)q;              /* 0..8; 8 is the smallest normal 0x08 */
        return (uint8_t)(sign | (uint8_t)code);
    }
    e = ilogbf(a);                          /* a in [2^e, 2^(e+1)) , e in [-6, 8] */
    q = nearbyintf(ldexpf(a, 3 - e));       /* in [8, 16] */
    if (q >= 16.0f) {
        q = 8.0f;
        e += 1;
    }
    if (e > 8 || (e == 8 && q > 14.0f)) {
        return (uint8_t)(sign | 0x7e);
    }
    code = ((e + 7) << 3) | ((int)q - 8);
    return (uint8_t)(sign | (uint8_t)code);
}

/* ---------------------------------------------------------------- CPU executor GEMM */

typedef struct {
    const float* a;
    const float* b;
    float* c;
    size_t k;
    size_t n;
    size_t row_begin;
    size_t row_end;
} orc_rows_job;

/* Order of operations of reference compiler_api.c:1747-1781: each output row
 * is zeroed, then k runs ascending (blocked by 64, which leaves the order
 * unchanged) and every column receives c += a[r,k] * b[k,c], the product
 * rounded to fp32 before the add (the file is built with -ffp-contract=off). */
static void orc_rows(const orc_rows_job* job) {
    size_t r;
    for (r = job->row_begin; r < job->row_end; ++r) {
        const float* arow = job->a + r * job->k;
        float* crow = job->c + r * job->n;
        size_t kk;
        memset(crow, 0, job->n * sizeof(float));
        for (kk = 0; kk < job->k; ++kk) {
            const float av = arow[kk];
            const float* brow = job->b + kk * job->n;
            size_t col;
            for (col = 0; col < job->n; ++col) {
                crow[col] += av * brow[col];
            }
        }
    }
}

static void* orc_rows_worker(void* arg) {
    orc_rows(arg);
    return NULL;
}

/* Row split across threads as reference compiler_api.c:1783-1812: the count
 * is capped at 32 and at m, and forced to 1 when m < 8. */
void orc_matmul_f32(const float* a, const float* b, float* c,
                    size_t m, size_t k, size_t n, int threads) {
    size_t t_count = threads > 0 ? (size_t)threads : 1;
    size_t per;
    size_t t;
    pthread_t tids[32];
    orc_rows_job jobs[32];
    size_t launched = 0;
    if (t_count > 32) {
        t_count = 32;
    }
    if (t_count > m) {
        t_count = m;
    }
    if (m < 8) {
        t_count = 1;
    }
    if (t_count <= 1) {
        orc_rows_job one = {a, b, c, k, n, 0, m};
        orc_rows(&one);
        return;
    }
    per = (m + t_count - 1) / t_count;
    for (t = 0; t < t_count; ++t) {
        size_t r0 = t * per;
        size_t r1 = r0 + per > m ? m : r0 + per;
        if (r0 >= m) {
            break;
        }
        jobs[t].a = a;
        jobs[t].b = b;
        jobs[t].c = c;
        jobs[t].k = k;
        jobs[t].n = n;
        jobs[t].row_begin = r0;
        jobs[t].row_end = r1;
        if (pthread_create(&tids[t], NULL, orc_rows_worker, &jobs[t]) != 0) {
            orc_rows(&jobs[t]);
            continue;
        }
        launched |= ((size_t)1) << t;
    }
    for (t = 0; t < t_count; ++t) {
        if (launched & (((size_t)1) << t)) {
            pthread_join(tids[t], NULL);
        }
    }
}

/* Add modes of reference cuda_backend.c:1201-1230 / :1697-1731:
 * 1 = MATRIX [M,N], 2 = ROW_BIAS [N] broadcast over rows, 3 = SCALAR [1]. */
void orc_add_epilogue(float* out, const float* addend, size_t m, size_t n, int mode) {
    size_t r, c;
    for (r = 0; r < m; ++r) {
        for (c = 0; c < n; ++c) {
            float v;
            if (mode == 1) {
                v = addend[r * n + c];
            } else if (mode == 2) {
                v = addend[c];
            } else {
                v = addend[0];
            }
            out[r * n + c] += v;
        }
    }
}

void orc_relu(float* out, size_t count) {
    size_t i;
    for (i = 0; i < count; ++i) {
        out[i] = out[i] > 0.0f ? out[i] : 0.0f;
    }
}

/* bf16 GEMM reference for rows [r0, r1): decode A rows and B (stored [K,N]
 * when b_trans == 0, [N,K] when b_trans == 1) to fp32, then the CPU executor
 * arithmetic. c receives (r1-r0) x n fp32 values. */
void orc_gemm_bf16(const uint16_t* a, const uint16_t* b, float* c,
                   size_t m, size_t n, size_t k, int b_trans,
                   size_t r0, size_t r1, int threads) {
    size_t rows = r1 - r0;
    float* af = (float*)malloc(rows * k * sizeof(float));
    float* bf = (float*)malloc(k * n * sizeof(float));
    size_t i, j;
    (void)m;
    if (!af || !bf) {
        free(af);
        free(bf);
        return;
    }
    for (i = 0; i < rows * k; ++i) {
        af[i] = orc_bf16_to_f32(a[r0 * k + i]);
    }
    if (b_trans) {
        for (j = 0; j < n; ++j) {
            for (i = 0; i < k; ++i) {
                bf[i * n + j] = orc_bf16_to_f32(b[j * k + i]);
            }
        }
    } else {
        for (i = 0; i < k * n; ++i) {
            bf[i] = orc_bf16_to_f32(b[i]);
        }
    }
    orc_matmul_f32(af, bf, c, rows, k, n, threads);
    free(af);
    free(bf);
}

/* ---------------------------------------------------------------- attention */

/* O[b,h,i,:] = sum_j p_ij V[b,h,j,:], p = softmax_j(s_ij), s_ij = scale * Q_i.K_j
 * over j <= i when causal (all j otherwise). Inputs/outputs fp32 [B,H,S,D];
 * only the (b,h) pairs with index in [bh0, bh1) are computed (flattened b*H+h). */
void orc_attention_f32(const float* q, const float* k, const float* v, float* o,
                       int B, int H, int S, int D, int causal, float scale,
                       int bh0, int bh1) {
    float* s = (float*)malloc((size_t)S * sizeof(float));
    int bh, i, j, d;
    (void)B;
    (void)H;
    if (!s) {
        return;
    }
    for (bh = bh0; bh < bh1; ++bh) {
        const float* qb = q + (size_t)bh * S * D;
        const float* kb = k + (size_t)bh * S * D;
        const float* vb = v + (size_t)bh * S * D;
        float* ob = o + (size_t)bh * S * D;
        for (i = 0; i < S; ++i) {
            int jend = causal ? i + 1 : S;
            float mx = -INFINITY;
            float denom = 0.0f;
            for (j = 0; j < jend; ++j) {
                float acc = 0.0f;
                for (d = 0; d < D; ++d) {
                    acc += qb[(size_t)i * D + d] * kb[(size_t)j * D + d];
                }
                s[j] = acc * scale;
                if (s[j] > mx) {
                    mx = s[j];
                }
            }
            for (j = 0; j < jend; ++j) {
                s[j] = expf(s[j] - mx);
                denom += s[j];
            }
            for (d = 0; d < D; ++d) {
                float acc = 0.0f;
                for (j = 0; j < jend; ++j) {
                    acc += s[j] * vb[(size_t)j * D + d];
                }
                ob[(size_t)i * D + d] = acc / denom;
            }
        }
    }
    free(s);
}

/* ---------------------------------------------------------------- conv2d */

/* y[n,p,q,kk] = relu?(bias[kk] + sum_{r,s,c} x[n, p*sh-ph+r, q*sw-pw+s, c] * w[kk,r,s,c])
 * x NHWC, w KRSC, y NPQK, all fp32; images [n0, n1) only. */
void orc_conv2d_nhwc_f32(const float* x, const float* w, const float* bias, float* y,
                         int N, int H, int W, int C, int K, int R, int S,
                         int pad_h, int pad_w, int stride_h, int stride_w, int relu,
                         int n0, int n1) {
    int P = (H + 2 * pad_h - R) / stride_h + 1;
    int Q = (W + 2 * pad_w - S) / stride_w + 1;
    int n, p, qq, kk, r, s, c;
    (void)N;
    for (n = n0; n < n1; ++n) {
        for (p = 0; p < P; ++p) {
            for (qq = 0; qq < Q; ++qq) {
                float* yo = y + (((size_t)n * P + p) * Q + qq) * K;
                for (kk = 0; kk < K; ++kk) {
                    float acc = 0.0f;
                    for (r = 0; r < R; ++r) {
                        int ih = p * stride_h - pad_h + r;
                        if (ih < 0 || ih >= H) {
                            continue;
                        }
                        for (s = 0; s < S; ++s) {
                            int iw = qq * stride_w - pad_w + s;
                            const float* xi;
                            const float* wi;
                            if (iw < 0 || iw >= W) {
                                continue;
                            }
                            xi = x + (((size_t)n * H + ih) * W + iw) * C;
                            wi = w + (((size_t)kk * R + r) * S + s) * C;
                            for (c = 0; c < C; ++c) {
                                acc += xi[c] * wi[c];
                            }
                        }
                    }
                    if (bias) {
                        acc += bias[kk];
                    }
                    if (relu && acc < 0.0f) {
                        acc = 0.0f;
                    }
                    yo[kk] = acc;
                }
            }
        }
    }
}

/* ---------------------------------------------------------------- fp8 decode layer */

/* One weight-only fp8 layer: Y[m,n] = bf16( relu?( scale[n] * sum_k X[m,k] * e4m3(Wq[n,k]) ) ),
 * X bf16 [M,K], Wq [N,K] e4m3fn, Y bf16 [M,N]. Sum in fp32, k ascending.
 * orc_w8a16_layer_mt splits the output channels over `threads` threads (each
 * channel's arithmetic is the same as with one). */
typedef struct {
    const float* xf;
    const uint8_t* wq;
    const float* scale;
    const float* lut;
    uint16_t* y;
    int M, N, K, relu, n0, n1;
} orc_w8_job;

static void* orc_w8_cols(void* arg) {
    const orc_w8_job* j = (const orc_w8_job*)arg;
    int m, n, kk;
    for (n = j->n0; n < j->n1; ++n) {
        const uint8_t* wr = j->wq + (size_t)n * j->K;
        for (m = 0; m < j->M; ++m) {
            const float* xr = j->xf + (size_t)m * j->K;
            float acc = 0.0f;
            for (kk = 0; kk < j->K; ++kk) {
                acc += xr[kk] * j->lut[wr[kk]];
            }
            acc *= j->scale[n];
            if (j->relu && acc < 0.0f) {
                acc = 0.0f;
            }
            j->y[(size_t)m * j->N + n] = orc_f32_to_bf16(acc);
        }
    }
    return NULL;
}

void orc_w8a16_layer_mt(const uint16_t* x, const uint8_t* wq, const float* scale,
                        uint16_t* y, int M, int N, int K, int relu, int threads) {
    float lut[256];
    float* xf = (float*)malloc((size_t)M * K * sizeof(float));
    orc_w8_job jobs[64];
    pthread_t tid[64];
    int started[64];
    int i, t, per;
    if (!xf) {
        return;
    }
    for (i = 0; i < 256; ++i) {
        lut[i] = orc_e4m3_to_f32((uint8_t)i);
    }
    for (i = 0; i < M * K; ++i) {
        xf[i] = orc_bf16_to_f32(x[i]);
    }
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    if (threads > N) threads = N;
    per = (N + threads - 1) / threads;
    for (t = 0; t < threads; ++t) {
        orc_w8_job jb = {xf, wq, scale, lut, y, M, N, K, relu, t * per < N ? t * per : N,
                         (t + 1) * per < N ? (t + 1) * per : N};
        jobs[t] = jb;
        started[t] = threads > 1 && pthread_create(&tid[t], NULL, orc_w8_cols, &jobs[t]) == 0;
        if (!started[t]) {
            orc_w8_cols(&jobs[t]);
        }
    }
    for (t = 0; t < threads; ++t) {
        if (started[t]) {
            pthread_join(tid[t], NULL);
        }
    }
    free(xf);
}

void orc_w8a16_layer(const uint16_t* x, const uint8_t* wq, const float* scale,
                     uint16_t* y, int M, int N, int K, int relu) {
    orc_w8a16_layer_mt(x, wq, scale, y, M, N, K, relu, 1);
}

/* Per-output-channel quantization of a weight W[K,N] (row-major, as the
 * decode chain is specified) into Wq[N,K] e4m3fn with scale[n] = max_k|W[k,n]|/448
 * (scale 1 for an all-zero column). */
void orc_quantize_e4m3_per_col(const float* w, int K, int N, uint8_t* wq, float* scale) {
    int n, kk;
    for (n = 0; n < N; ++n) {
        float amax = 0.0f;
        float s;
        for (kk = 0; kk < K; ++kk) {
            float a = fabsf(w[(size_t)kk * N + n]);
            if (a > amax) {
                amax = a;
            }
        }
        s = amax > 0.0f ? amax / 448.0f : 1.0f;
        scale[n] = s;
        for (kk = 0; kk < K; ++kk) {
            wq[(size_t)n * K + kk] = orc_f32_to_e4m3(w[(size_t)kk * N + n] / s);
        }
    }
}

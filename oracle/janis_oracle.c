/*
 * janis_oracle.c -- TEST INFRASTRUCTURE ONLY (see janis_oracle.h).
 *
 * CPU restatement of the quantized-linear arithmetic of janis's Go CPU
 * backend. Compiled with -O2 -ffp-contract=off: a product and the add that
 * follows it round separately unless the code calls fmaf(), which is how the
 * Go compiler emits `a*b + c` on amd64 (GOAMD64=v1) and how the reference's
 * AVX2 assembly uses VFMADD231PS.
 */
#include "janis_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

static inline uint32_t code_at(const uint32_t *row, int64_t j, int bits) {
    const int vpw = 32 / bits;
    const uint32_t mask = (bits == 32) ? 0xFFFFFFFFu : ((1u << bits) - 1u);
    return (row[j / vpw] >> ((j % vpw) * bits)) & mask;
}

/* cpu/cpu_misc.go:134-161 */
void or_dequantize(const uint32_t *w, const float *s, const float *b, float *out,
                   int64_t rows, int64_t P, int64_t G, int group_size, int bits) {
    const int64_t in = P * (32 / bits);
    for (int64_t r = 0; r < rows; r++) {
        const uint32_t *wr = w + r * P;
        const float *sr = s + r * G, *br = b + r * G;
        float *o = out + r * in;
        for (int64_t j = 0; j < in; j++) {
            const int64_t g = j / group_size;
            const float t = (float)code_at(wr, j, bits) * sr[g];
            o[j] = t + br[g];
        }
    }
}

/* cpu/qmv_test.go:11-29 */
float or_qchannel4_ref(const uint32_t *w, const float *x, const float *s, const float *b,
                       int groups, int words_per_group) {
    float acc = 0.0f;
    int64_t xi = 0, wp = 0;
    for (int g = 0; g < groups; g++) {
        float sum_xq = 0.0f, sum_x = 0.0f;
        for (int wc = 0; wc < words_per_group; wc++) {
            const uint32_t word = w[wp++];
            for (int v = 0; v < 8; v++) {
                const float xv = x[xi++];
                const float p = xv * (float)((word >> (4 * v)) & 0xFu);
                sum_xq = sum_xq + p;
                sum_x = sum_x + xv;
            }
        }
        const float t1 = s[g] * sum_xq;
        const float t2 = b[g] * sum_x;
        acc = acc + (t1 + t2);
    }
    return acc;
}

/* cpu/qmv_amd64.s:28-81, one lane per nibble position. */
float or_qchannel4_avx2_order(const uint32_t *w, const float *x, const float *s, const float *b,
                              int groups, int words_per_group) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int g = 0; g < groups; g++) {
        float sxq[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        float sx[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int wc = 0; wc < words_per_group; wc++) {
            const uint32_t word = *w++;
            for (int l = 0; l < 8; l++) {
                const float q = (float)((word >> (4 * l)) & 0xFu);
                sxq[l] = fmaf(q, x[l], sxq[l]); /* :53 VFMADD231PS */
                sx[l] = sx[l] + x[l];           /* :54 VADDPS */
            }
            x += 8;
        }
        for (int l = 0; l < 8; l++) {
            acc[l] = fmaf(s[g], sxq[l], acc[l]); /* :68 */
            acc[l] = fmaf(b[g], sx[l], acc[l]);  /* :69 */
        }
    }
    /* :73-79: lo4 + hi4, then two horizontal pair-adds. */
    const float t0 = acc[0] + acc[4], t1 = acc[1] + acc[5];
    const float t2 = acc[2] + acc[6], t3 = acc[3] + acc[7];
    return (t0 + t1) + (t2 + t3);
}

/* Go's parWork/parallelFor chunk layout (cpu/cpu.go:37-79): returns the
 * number of chunks and the chunk length. */
static int64_t go_chunks(int64_t n, int64_t unit, int workers, int64_t *chunk) {
    if (n <= 0) {
        *chunk = 0;
        return 0;
    }
    if (n * unit < (1 << 16) || workers <= 1) {
        *chunk = n;
        return 1;
    }
    int64_t wk = workers;
    if (wk > n) wk = n;
    *chunk = (n + wk - 1) / wk;
    return (n + *chunk - 1) / *chunk;
}

/* cpu/cpu_misc.go:277-347, for one chunk [os, oe). */
static void blocked_go_chunk(const float *x0, const uint32_t *w, const float *s, const float *b,
                             float *y, int64_t os, int64_t oe, int64_t P, int64_t G, int wpg) {
    int64_t o = os;
    for (; o + 4 <= oe; o += 4) {
        const uint32_t *wp[4] = {w + o * P, w + (o + 1) * P, w + (o + 2) * P, w + (o + 3) * P};
        float acc[4] = {0, 0, 0, 0};
        int64_t xi = 0;
        for (int64_t g = 0; g < G; g++) {
            float q[4] = {0, 0, 0, 0};
            float sx = 0.0f;
            for (int wc = 0; wc < wpg; wc++) {
                const float *a = x0 + xi;
                xi += 8;
                for (int c = 0; c < 4; c++) {
                    const uint32_t word = *wp[c]++;
                    /* left-associated sum of the 8 rounded products */
                    float e = a[0] * (float)(word & 0xFu);
                    for (int v = 1; v < 8; v++) e = e + a[v] * (float)((word >> (4 * v)) & 0xFu);
                    q[c] = q[c] + e;
                }
                float t = a[0];
                for (int v = 1; v < 8; v++) t = t + a[v];
                sx = sx + t;
            }
            for (int c = 0; c < 4; c++) {
                const int64_t sb = (o + c) * G + g;
                const float t1 = s[sb] * q[c];
                const float t2 = b[sb] * sx;
                acc[c] = acc[c] + (t1 + t2);
            }
        }
        for (int c = 0; c < 4; c++) y[o + c] = acc[c];
    }
    for (; o < oe; o++) { /* remainder: two lanes, even and odd nibbles */
        const uint32_t *wp = w + o * P;
        float acc = 0.0f;
        int64_t xi = 0;
        for (int64_t g = 0; g < G; g++) {
            float xq0 = 0, xq1 = 0, sx0 = 0, sx1 = 0;
            for (int wc = 0; wc < wpg; wc++) {
                const uint32_t word = *wp++;
                const float *a = x0 + xi;
                xi += 8;
                float e0 = a[0] * (float)(word & 0xFu);
                e0 = e0 + a[2] * (float)((word >> 8) & 0xFu);
                e0 = e0 + a[4] * (float)((word >> 16) & 0xFu);
                e0 = e0 + a[6] * (float)((word >> 24) & 0xFu);
                float e1 = a[1] * (float)((word >> 4) & 0xFu);
                e1 = e1 + a[3] * (float)((word >> 12) & 0xFu);
                e1 = e1 + a[5] * (float)((word >> 20) & 0xFu);
                e1 = e1 + a[7] * (float)((word >> 28) & 0xFu);
                xq0 = xq0 + e0;
                xq1 = xq1 + e1;
                sx0 = sx0 + (((a[0] + a[2]) + a[4]) + a[6]);
                sx1 = sx1 + (((a[1] + a[3]) + a[5]) + a[7]);
            }
            const int64_t sb = o * G + g;
            const float t1 = s[sb] * (xq0 + xq1);
            const float t2 = b[sb] * (sx0 + sx1);
            acc = acc + (t1 + t2);
        }
        y[o] = acc;
    }
}

void or_qmv_blocked_go(const float *x, const uint32_t *w, const float *s, const float *b,
                       float *y, int64_t N, int64_t K, int group_size, int workers) {
    const int64_t P = K / 8, G = K / group_size;
    const int wpg = group_size / 8;
    int64_t chunk;
    const int64_t nchunks = go_chunks(N, K, workers, &chunk);
    for (int64_t c = 0; c < nchunks; c++) {
        const int64_t os = c * chunk;
        const int64_t oe = (os + chunk < N) ? os + chunk : N;
        blocked_go_chunk(x, w, s, b, y, os, oe, P, G, wpg);
    }
}

/* cpu/cpu_misc.go:350-375 */
void or_qmv_generic(const float *x, const uint32_t *w, const float *s, const float *b,
                    float *y, int64_t N, int64_t K, int group_size, int bits) {
    const int vpw = 32 / bits;
    const uint32_t mask = (bits == 32) ? 0xFFFFFFFFu : ((1u << bits) - 1u);
    const int64_t P = K / vpw, G = K / group_size;
    const int wpg = group_size / vpw;
    for (int64_t o = 0; o < N; o++) {
        const uint32_t *wp = w + o * P;
        float acc = 0.0f;
        int64_t xi = 0;
        for (int64_t g = 0; g < G; g++) {
            float sum_xq = 0.0f, sum_x = 0.0f;
            for (int wc = 0; wc < wpg; wc++) {
                const uint32_t word = *wp++;
                for (int v = 0; v < vpw; v++) {
                    const float xv = x[xi++];
                    const float p = xv * (float)((word >> (v * bits)) & mask);
                    sum_xq = sum_xq + p;
                    sum_x = sum_x + xv;
                }
            }
            const float t1 = s[o * G + g] * sum_xq;
            const float t2 = b[o * G + g] * sum_x;
            acc = acc + (t1 + t2);
        }
        y[o] = acc;
    }
}

/* cpu/cpu_misc.go:378-399 */
void or_qmm_wbuf(const float *x, int64_t rows, const uint32_t *w, const float *s, const float *b,
                 float *y, int64_t N, int64_t K, int group_size, int bits) {
    const int64_t P = K / (32 / bits), G = K / group_size;
    float *wbuf = (float *)malloc((size_t)K * sizeof(float));
    if (!wbuf) abort();
    for (int64_t o = 0; o < N; o++) {
        const uint32_t *wr = w + o * P;
        for (int64_t i = 0; i < K; i++) {
            const int64_t g = i / group_size;
            const float t = (float)code_at(wr, i, bits) * s[o * G + g];
            wbuf[i] = t + b[o * G + g];
        }
        for (int64_t r = 0; r < rows; r++) {
            const float *xr = x + r * K;
            float acc = 0.0f;
            for (int64_t i = 0; i < K; i++) {
                const float p = xr[i] * wbuf[i];
                acc = acc + p;
            }
            y[r * N + o] = acc;
        }
    }
    free(wbuf);
}

/* cpu/cpu_misc.go:232-400 as dispatched on amd64. */
void or_quant_matmul(const float *x, int64_t rows, const uint32_t *w, const float *s,
                     const float *b, float *y, int64_t N, int64_t K, int group_size, int bits,
                     int simd) {
    const int vpw = 32 / bits;
    if (rows == 1 && group_size % vpw == 0) {
        if (bits == 4 && simd) {
            const int64_t P = K / 8, G = K / group_size;
            for (int64_t o = 0; o < N; o++)
                y[o] = or_qchannel4_avx2_order(w + o * P, x, s + o * G, b + o * G, (int)G,
                                               group_size / 8);
            return;
        }
        if (bits == 4) {
            or_qmv_blocked_go(x, w, s, b, y, N, K, group_size, 1);
            return;
        }
        or_qmv_generic(x, w, s, b, y, N, K, group_size, bits);
        return;
    }
    or_qmm_wbuf(x, rows, w, s, b, y, N, K, group_size, bits);
}

/* cpu/cpu_misc.go:178-230 */
int or_gather_quant_matmul(const float *x, int64_t n_lead, int64_t A, const uint32_t *w,
                           const float *s, const float *b, int64_t E, const int32_t *idx,
                           int64_t k_slots, float *y, int64_t N, int64_t K, int group_size,
                           int bits, int simd) {
    const int64_t P = K / (32 / bits), G = K / group_size;
    const int64_t npairs = n_lead * k_slots;
    for (int64_t i = 0; i < npairs; i++)
        if (idx[i] < 0 || idx[i] >= E) return -1;
    int64_t *src = (int64_t *)malloc((size_t)(npairs + 1) * sizeof(int64_t));
    int64_t *dst = (int64_t *)malloc((size_t)(npairs + 1) * sizeof(int64_t));
    float *xb = (float *)malloc((size_t)(npairs + 1) * (size_t)K * sizeof(float));
    float *yb = (float *)malloc((size_t)(npairs + 1) * (size_t)N * sizeof(float));
    if (!src || !dst || !xb || !yb) abort();
    for (int64_t e = 0; e < E; e++) {
        /* slots routed to e, in (lead, slot) order (:197-209) */
        int64_t R = 0;
        for (int64_t l = 0; l < n_lead; l++)
            for (int64_t k = 0; k < k_slots; k++)
                if (idx[l * k_slots + k] == e) {
                    const int64_t a = (A == 1) ? 0 : k;
                    src[R] = (l * A + a) * K;
                    dst[R] = (l * k_slots + k) * N;
                    R++;
                }
        if (R == 0) continue;
        for (int64_t r = 0; r < R; r++) memcpy(xb + r * K, x + src[r], (size_t)K * sizeof(float));
        or_quant_matmul(xb, R, w + e * N * P, s + e * N * G, b + e * N * G, yb, N, K, group_size,
                        bits, simd);
        for (int64_t r = 0; r < R; r++) memcpy(y + dst[r], yb + r * N, (size_t)N * sizeof(float));
    }
    free(src);
    free(dst);
    free(xb);
    free(yb);
    return 0;
}

/* ---- CPU baseline: the AVX2 kernel over parallelFor chunks ---------------- */

typedef struct {
    const float *x;
    const uint32_t *w;
    const float *s, *b;
    float *y;
    int64_t os, oe, P, G;
    int wpg, avx2;
} qmv_job;

static void *qmv_job_run(void *arg) {
    const qmv_job *j = (const qmv_job *)arg;
    for (int64_t o = j->os; o < j->oe; o++) {
        const uint32_t *wr = j->w + o * j->P;
        const float *sr = j->s + o * j->G, *br = j->b + o * j->G;
        j->y[o] = j->avx2 ? or_qchannel4_avx2(wr, j->x, sr, br, (int)j->G, j->wpg)
                          : or_qchannel4_avx2_order(wr, j->x, sr, br, (int)j->G, j->wpg);
    }
    return NULL;
}

/* cpu/cpu_misc.go:265-276 over cpu/cpu.go:37-79 */
int or_qmv_avx2_parallel(const float *x, const uint32_t *w, const float *s, const float *b,
                         float *y, int64_t N, int64_t K, int group_size, int workers) {
    int64_t chunk;
    const int64_t n = go_chunks(N, K, workers, &chunk);
    if (n == 0) return 0;
    qmv_job *jobs = (qmv_job *)calloc((size_t)n, sizeof(qmv_job));
    pthread_t *th = (pthread_t *)calloc((size_t)n, sizeof(pthread_t));
    if (!jobs || !th) abort();
    const int avx2 = or_have_avx2_fma();
    for (int64_t c = 0; c < n; c++) {
        jobs[c].x = x;
        jobs[c].w = w;
        jobs[c].s = s;
        jobs[c].b = b;
        jobs[c].y = y;
        jobs[c].os = c * chunk;
        jobs[c].oe = (c * chunk + chunk < N) ? c * chunk + chunk : N;
        jobs[c].P = K / 8;
        jobs[c].G = K / group_size;
        jobs[c].wpg = group_size / 8;
        jobs[c].avx2 = avx2;
    }
    /* every chunk but the last on its own thread, the last on the caller */
    for (int64_t c = 0; c + 1 < n; c++)
        if (pthread_create(&th[c], NULL, qmv_job_run, &jobs[c]) != 0) abort();
    qmv_job_run(&jobs[n - 1]);
    for (int64_t c = 0; c + 1 < n; c++) pthread_join(th[c], NULL);
    free(jobs);
    free(th);
    return (int)n;
}

/* qwen/moe.go:501-511 */
int or_moe_apply(const float *x, int64_t n_tok, const uint32_t *wg, const float *sg,
                 const float *bg, const uint32_t *wu, const float *su, const float *bu,
                 const uint32_t *wd, const float *sd, const float *bd, int64_t E, int64_t H,
                 int64_t I, const int32_t *idx, const float *scores, int64_t k_slots, float *out,
                 int group_size, int simd) {
    const int64_t np = n_tok * k_slots;
    float *g = (float *)malloc((size_t)(np * I + 1) * sizeof(float));
    float *u = (float *)malloc((size_t)(np * I + 1) * sizeof(float));
    float *d = (float *)malloc((size_t)(np * H + 1) * sizeof(float));
    if (!g || !u || !d) abort();
    int rc = or_gather_quant_matmul(x, n_tok, 1, wg, sg, bg, E, idx, k_slots, g, I, H, group_size, 4, simd);
    if (rc == 0)
        rc = or_gather_quant_matmul(x, n_tok, 1, wu, su, bu, E, idx, k_slots, u, I, H, group_size, 4, simd);
    if (rc == 0) {
        for (int64_t i = 0; i < np * I; i++) {
            const float v = g[i];
            const float e = (float)exp((double)(-v));
            const float silu = v / (1.0f + e);
            g[i] = silu * u[i];
        }
        rc = or_gather_quant_matmul(g, n_tok, k_slots, wd, sd, bd, E, idx, k_slots, d, H, I, group_size, 4,
                                    simd);
    }
    if (rc == 0) {
        for (int64_t t = 0; t < n_tok; t++)
            for (int64_t j = 0; j < H; j++) {
                float acc = 0.0f;
                for (int64_t k = 0; k < k_slots; k++) {
                    const float p = d[(t * k_slots + k) * H + j] * scores[t * k_slots + k];
                    acc = acc + p;
                }
                const float mean = acc / (float)k_slots;
                out[t * H + j] = mean * (float)k_slots;
            }
    }
    free(g);
    free(u);
    free(d);
    return rc;
}

/* ---- MoE routing helpers ----------------------------------------------- */

/* qwen/moe.go:420-444 */
void or_topk(const float *row, int n, int k, int32_t *idx, float *val) {
    int *order = (int *)malloc((size_t)n * sizeof(int));
    if (!order) abort();
    for (int i = 0; i < n; i++) order[i] = i;
    for (int i = 0; i < k && i < n; i++) {
        int best = i;
        for (int j = i + 1; j < n; j++)
            if (row[order[j]] > row[order[best]]) best = j;
        const int t = order[i];
        order[i] = order[best];
        order[best] = t;
    }
    if (k > n) k = n;
    for (int i = 0; i < k; i++) {
        idx[i] = order[i];
        val[i] = row[order[i]];
    }
    free(order);
}

/* cpu/cpu.go:461-499 for one contiguous row */
void or_softmax_row(const float *x, float *out, int n) {
    float mx = -INFINITY;
    for (int i = 0; i < n; i++)
        if (x[i] > mx) mx = x[i];
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        const float e = (float)exp((double)(x[i] - mx));
        out[i] = e;
        sum = sum + e;
    }
    for (int i = 0; i < n; i++) out[i] = out[i] / sum;
}

/* ---- decode-step operators ------------------------------------------------ */

/* cpu/cpu_ops.go:144-162: per row, ss = sum x^2 in index order (fp32),
 * inv = 1 / fl32(sqrt(fl64(ss/d + eps))), out = x * inv * w (left to right). */
void or_rms_norm(const float *x, const float *w, float *out, int64_t rows, int64_t d, float eps) {
    for (int64_t r = 0; r < rows; r++) {
        const float *xr = x + r * d;
        float ss = 0.0f;
        for (int64_t i = 0; i < d; i++) {
            const float v = xr[i];
            ss = ss + v * v;
        }
        const float inv = 1.0f / (float)sqrt((double)(ss / (float)d + eps));
        for (int64_t i = 0; i < d; i++) {
            const float t = xr[i] * inv;
            out[r * d + i] = t * w[i];
        }
    }
}

/* cpu/cpu_attn.go:13-62. x holds rows of D features; the row's position is
 * offset + (r % L). inv[i] = fl32(base^(-2i/dims)) (RoPE) or 1/freqs[i]
 * (RoPEFreqs, freqs != NULL). Non-traditional pairs (i, i+dims/2), traditional
 * (2i, 2i+1); features past `dims` pass through. */
void or_rope(const float *x, float *out, int64_t rows, int64_t L, int64_t D, int dims, int traditional,
             float base, float scale, int64_t offset, const float *freqs) {
    const int half = dims / 2;
    float *inv = (float *)malloc((size_t)(half > 0 ? half : 1) * sizeof(float));
    if (!inv) abort();
    for (int i = 0; i < half; i++)
        inv[i] = freqs ? 1.0f / freqs[i] : (float)pow((double)base, -(double)(2 * i) / (double)dims);
    memcpy(out, x, (size_t)(rows * D) * sizeof(float));
    for (int64_t r = 0; r < rows; r++) {
        const float pos = (float)(offset + r % L);
        const int64_t o = r * D;
        for (int i = 0; i < half; i++) {
            const float theta = pos * scale * inv[i];
            const float c = (float)cos((double)theta);
            const float s = (float)sin((double)theta);
            const int64_t i0 = traditional ? o + 2 * i : o + i;
            const int64_t i1 = traditional ? o + 2 * i + 1 : o + i + half;
            const float a = x[i0], b2 = x[i1];
            const float ac = a * c, bs = b2 * s, as_ = a * s, bc = b2 * c;
            out[i0] = ac - bs;
            out[i1] = as_ + bc;
        }
    }
    free(inv);
}

/* cpu/cpu_attn.go:64-119: q [B, Hq, Lq, Dh], k/v [B, Hk, Lk, Dh] contiguous,
 * out [B, Hq, Lq, Dh]. Query head h reads kv head h / (Hq/Hk). With causal, row
 * i sees keys j <= (Lk - Lq) + i. Scores are fp32 dots in index order times
 * scale; softmax with exp in double; out = sum_j (e_j / sum) * v_j in key order. */
void or_sdpa(const float *q, const float *k, const float *v, float *out, int64_t B, int64_t Hq, int64_t Hk,
             int64_t Lq, int64_t Lk, int64_t Dh, float scale, int causal) {
    const int64_t group = Hq / Hk, delta = Lk - Lq;
    float *sc = (float *)malloc((size_t)(Lk > 0 ? Lk : 1) * sizeof(float));
    if (!sc) abort();
    for (int64_t bi = 0; bi < B; bi++)
        for (int64_t h = 0; h < Hq; h++) {
            const int64_t hk = h / group;
            for (int64_t i = 0; i < Lq; i++) {
                const int64_t limit = causal ? delta + i + 1 : Lk;
                const float *qr = q + ((bi * Hq + h) * Lq + i) * Dh;
                float mx = -INFINITY;
                for (int64_t j = 0; j < limit; j++) {
                    const float *kr = k + ((bi * Hk + hk) * Lk + j) * Dh;
                    float s = 0.0f;
                    for (int64_t d = 0; d < Dh; d++) s = s + qr[d] * kr[d];
                    s = s * scale;
                    sc[j] = s;
                    if (s > mx) mx = s;
                }
                float sum = 0.0f;
                for (int64_t j = 0; j < limit; j++) {
                    const float e = (float)exp((double)(sc[j] - mx));
                    sc[j] = e;
                    sum = sum + e;
                }
                float *orow = out + ((bi * Hq + h) * Lq + i) * Dh;
                for (int64_t d = 0; d < Dh; d++) {
                    float acc = 0.0f;
                    for (int64_t j = 0; j < limit; j++) {
                        const float *vr = v + ((bi * Hk + hk) * Lk + j) * Dh;
                        acc = acc + (sc[j] / sum) * vr[d];
                    }
                    orow[d] = acc;
                }
            }
        }
    free(sc);
}

/* cpu/cpu.go:327-329 */
void or_silu(const float *x, float *out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = x[i] / (1.0f + (float)exp((double)(-x[i])));
}

/* cpu/cpu_misc.go:91-121 over the last axis: first index of the maximum
 * (strict '>'), 0 when no element beats -inf. */
void or_argmax(const float *x, int64_t rows, int64_t n, int32_t *out) {
    for (int64_t r = 0; r < rows; r++) {
        float best = -INFINITY;
        int32_t bi = 0;
        for (int64_t i = 0; i < n; i++)
            if (x[r * n + i] > best) best = x[r * n + i], bi = (int32_t)i;
        out[r] = bi;
    }
}

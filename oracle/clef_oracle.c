/*
 * clef_oracle.c -- CPU F32 restatement of the clef-rs hybrid prefill path.
 *
 * TEST INFRASTRUCTURE ONLY (parity checker and CPU baseline); see
 * clef_oracle.h for the pinning of each function.  Compiled with
 * -ffp-contract=off so that every multiply and add rounds separately, as the
 * reference's tensor graph does.
 */
#include "clef_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ */
/* f16 helpers                                                          */
/* ------------------------------------------------------------------ */
uint16_t oracle_f32_to_f16(float x) {
    union { float f; uint32_t u; } v = {x};
    uint32_t u = v.u;
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t absu = u & 0x7fffffffu;
    if (absu >= 0x7f800000u) { /* inf or nan */
        return (uint16_t)(sign | 0x7c00u | (absu > 0x7f800000u ? 0x200u : 0u));
    }
    if (absu >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* overflow to inf */
    if (absu < 0x38800000u) {                                    /* subnormal or zero */
        /* value = absu as float; f16 subnormal unit is 2^-24 */
        union { uint32_t u; float f; } a = {absu};
        float scaled = a.f * 16777216.0f; /* exact: power of two scaling */
        /* round to nearest even integer */
        float r = rintf(scaled);
        return (uint16_t)(sign | (uint32_t)r);
    }
    uint32_t exp = (absu >> 23) - 127 + 15;
    uint32_t mant = absu & 0x7fffffu;
    uint32_t half = (exp << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) half += 1u;
    return (uint16_t)(sign | half);
}

float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t mant = h & 0x3ffu;
    union { uint32_t u; float f; } v;
    if (exp == 0) {
        float m = (float)mant * (1.0f / 16777216.0f);
        return sign ? -m : m;
    } else if (exp == 31) {
        v.u = sign | 0x7f800000u | (mant << 13);
    } else {
        v.u = sign | ((exp - 15 + 127) << 23) | (mant << 13);
    }
    return v.f;
}

void oracle_round_f16(float* x, size_t n) {
    for (size_t i = 0; i < n; ++i) x[i] = oracle_f16_to_f32(oracle_f32_to_f16(x[i]));
}

static int g_threads = 0;
void oracle_set_threads(int n) { g_threads = n; }
int oracle_get_threads(void) {
#ifdef _OPENMP
    return g_threads > 0 ? g_threads : omp_get_max_threads();
#else
    return 1;
#endif
}
#define OMP_THREADS num_threads(oracle_get_threads())

/* ------------------------------------------------------------------ */
/* Gated delta rule, per token (qwen.rs:826-882)                        */
/* ------------------------------------------------------------------ */

/* l2(x) = x / sqrt(sum(x^2) + 1e-6), qwen.rs:837-840. */
static void l2_row(const float* x, int n, float* y) {
    float s = 0.0f;
    for (int i = 0; i < n; ++i) s += x[i] * x[i];
    float root = sqrtf(s + 1e-6f);
    for (int i = 0; i < n; ++i) y[i] = x[i] / root;
}

int oracle_delta_recurrence(const float* q, const float* k, const float* v, const float* g,
                            const float* beta, int T, int H, int dk, int dv,
                            const float* initial, int capture, float* out, float* captured,
                            float* final_state) {
    if (T < 1 || H < 1 || dk < 1 || dv < 1 || capture < 0 || capture > T) return -1;
    /* q <- l2(q) / sqrt(dk): Candle divides by an f64 scalar through an affine
     * multiply by the rounded reciprocal (qwen.rs:844; pointwise.metal:99). */
    const float qscale = (float)(1.0 / sqrt((double)dk));
    int h;
#pragma omp parallel for OMP_THREADS schedule(static)
    for (h = 0; h < H; ++h) {
        float* S = (float*)malloc(sizeof(float) * (size_t)dk * dv);
        float* kk = (float*)malloc(sizeof(float) * dk);
        float* qq = (float*)malloc(sizeof(float) * dk);
        float* mem = (float*)malloc(sizeof(float) * dv);
        float* delta = (float*)malloc(sizeof(float) * dv);
        if (initial)
            memcpy(S, initial + (size_t)h * dk * dv, sizeof(float) * (size_t)dk * dv);
        else
            memset(S, 0, sizeof(float) * (size_t)dk * dv);
        for (int t = 0; t < T; ++t) {
            const size_t row = (size_t)t * H + h;
            l2_row(k + row * dk, dk, kk);
            l2_row(q + row * dk, dk, qq);
            for (int i = 0; i < dk; ++i) qq[i] = qq[i] * qscale;
            /* state <- state * exp(g)                         qwen.rs:871 */
            const float decay = expf(g[row]);
            for (size_t i = 0; i < (size_t)dk * dv; ++i) S[i] = S[i] * decay;
            /* memory = sum_k state[k,:] * key[k]               qwen.rs:872 */
            for (int j = 0; j < dv; ++j) mem[j] = 0.0f;
            for (int i = 0; i < dk; ++i)
                for (int j = 0; j < dv; ++j) mem[j] = mem[j] + S[(size_t)i * dv + j] * kk[i];
            /* delta = (v - memory) * beta                       qwen.rs:873-874 */
            const float b = beta[row];
            for (int j = 0; j < dv; ++j) delta[j] = (v[row * dv + j] - mem[j]) * b;
            /* state <- state + key (x) delta                    qwen.rs:875 */
            for (int i = 0; i < dk; ++i)
                for (int j = 0; j < dv; ++j)
                    S[(size_t)i * dv + j] = S[(size_t)i * dv + j] + kk[i] * delta[j];
            /* o_t = sum_k state[k,:] * query[k]                  qwen.rs:876 */
            float* o = out + row * dv;
            for (int j = 0; j < dv; ++j) o[j] = 0.0f;
            for (int i = 0; i < dk; ++i)
                for (int j = 0; j < dv; ++j) o[j] = o[j] + S[(size_t)i * dv + j] * qq[i];
            /* capture after token i+1 == capture                qwen.rs:877-879 */
            if (captured && capture == t + 1)
                memcpy(captured + (size_t)h * dk * dv, S, sizeof(float) * (size_t)dk * dv);
        }
        if (final_state)
            memcpy(final_state + (size_t)h * dk * dv, S, sizeof(float) * (size_t)dk * dv);
        free(S); free(kk); free(qq); free(mem); free(delta);
    }
    return 0;
}

static void l2_row_f64(const double* x, int n, double* y) {
    double s = 0.0;
    for (int i = 0; i < n; ++i) s += x[i] * x[i];
    double root = sqrt(s + 1e-6);
    for (int i = 0; i < n; ++i) y[i] = x[i] / root;
}

int oracle_delta_recurrence_f64(const double* q, const double* k, const double* v,
                                const double* g, const double* beta, int T, int H, int dk,
                                int dv, const double* initial, double* out, double* final_state) {
    if (T < 1 || H < 1 || dk < 1 || dv < 1) return -1;
    const double qscale = 1.0 / sqrt((double)dk);
    double* S = (double*)malloc(sizeof(double) * (size_t)dk * dv);
    double* kk = (double*)malloc(sizeof(double) * dk);
    double* qq = (double*)malloc(sizeof(double) * dk);
    double* delta = (double*)malloc(sizeof(double) * dv);
    for (int h = 0; h < H; ++h) {
        if (initial)
            memcpy(S, initial + (size_t)h * dk * dv, sizeof(double) * (size_t)dk * dv);
        else
            memset(S, 0, sizeof(double) * (size_t)dk * dv);
        for (int t = 0; t < T; ++t) {
            const size_t row = (size_t)t * H + h;
            l2_row_f64(k + row * dk, dk, kk);
            l2_row_f64(q + row * dk, dk, qq);
            for (int i = 0; i < dk; ++i) qq[i] *= qscale;
            const double decay = exp(g[row]);
            for (size_t i = 0; i < (size_t)dk * dv; ++i) S[i] *= decay;
            for (int j = 0; j < dv; ++j) {
                double m = 0.0;
                for (int i = 0; i < dk; ++i) m += S[(size_t)i * dv + j] * kk[i];
                delta[j] = (v[row * dv + j] - m) * beta[row];
            }
            for (int i = 0; i < dk; ++i)
                for (int j = 0; j < dv; ++j) S[(size_t)i * dv + j] += kk[i] * delta[j];
            for (int j = 0; j < dv; ++j) {
                double o = 0.0;
                for (int i = 0; i < dk; ++i) o += S[(size_t)i * dv + j] * qq[i];
                out[row * dv + j] = o;
            }
        }
        if (final_state)
            memcpy(final_state + (size_t)h * dk * dv, S, sizeof(double) * (size_t)dk * dv);
    }
    free(S); free(kk); free(qq); free(delta);
    return 0;
}

/*
 * Chunkwise form (chunk.metal:10-164 with C a parameter; the same algebra as
 * transformers' chunk_gated_delta_rule).  Per chunk of C tokens with local
 * cumulative log-decay gam_r = sum_{j<=r} g_j, decay ratios are formed only for
 * c <= r as exp(sum_{c<j<=r} g_j) (never by dividing prefix products):
 *   A[r][c]  = beta_r (k_r . k_c) exp(gam_r - gam_c),  c < r
 *   Tm       = (I + A)^-1                      (forward substitution)
 *   Delta    = Tm diag(beta) (V - diag(exp gam) K S)
 *   O[r]     = exp(gam_r) q_r^T S + sum_{c<=r} (q_r . k_c) exp(gam_r - gam_c) Delta[c]
 *   S'       = exp(gam_last) S + sum_c exp(gam_last - gam_c) k_c (x) Delta[c]
 */
int oracle_delta_chunked_f64(const double* q, const double* k, const double* v, const double* g,
                             const double* beta, int T, int H, int dk, int dv, int C,
                             const double* initial, double* out, double* final_state) {
    if (T < 1 || H < 1 || dk < 1 || dv < 1 || C < 1) return -1;
    const double qscale = 1.0 / sqrt((double)dk);
    double* S = (double*)malloc(sizeof(double) * (size_t)dk * dv);
    double* Kn = (double*)malloc(sizeof(double) * (size_t)C * dk);
    double* Qn = (double*)malloc(sizeof(double) * (size_t)C * dk);
    double* gam = (double*)malloc(sizeof(double) * C);
    double* A = (double*)malloc(sizeof(double) * (size_t)C * C);
    double* Tm = (double*)malloc(sizeof(double) * (size_t)C * C);
    double* Y = (double*)malloc(sizeof(double) * (size_t)C * dv);
    double* D = (double*)malloc(sizeof(double) * (size_t)C * dv);
    double* Snew = (double*)malloc(sizeof(double) * (size_t)dk * dv);
    for (int h = 0; h < H; ++h) {
        if (initial)
            memcpy(S, initial + (size_t)h * dk * dv, sizeof(double) * (size_t)dk * dv);
        else
            memset(S, 0, sizeof(double) * (size_t)dk * dv);
        for (int t0 = 0; t0 < T; t0 += C) {
            const int n = (T - t0) < C ? (T - t0) : C;
            for (int r = 0; r < n; ++r) {
                const size_t row = (size_t)(t0 + r) * H + h;
                l2_row_f64(k + row * dk, dk, Kn + (size_t)r * dk);
                l2_row_f64(q + row * dk, dk, Qn + (size_t)r * dk);
                for (int i = 0; i < dk; ++i) Qn[(size_t)r * dk + i] *= qscale;
            }
            /* decay ratio exp(sum_{c<j<=r} g_j) for c <= r */
#define GROW(r) g[(size_t)(t0 + (r)) * H + h]
            for (int r = 0; r < n; ++r) gam[r] = (r ? gam[r - 1] : 0.0) + GROW(r);
            for (int r = 0; r < n; ++r)
                for (int c = 0; c < n; ++c) {
                    double a = 0.0;
                    if (c < r) {
                        double s = 0.0, dot = 0.0;
                        for (int j = c + 1; j <= r; ++j) s += GROW(j);
                        for (int i = 0; i < dk; ++i) dot += Kn[(size_t)r * dk + i] * Kn[(size_t)c * dk + i];
                        a = beta[(size_t)(t0 + r) * H + h] * dot * exp(s);
                    }
                    A[(size_t)r * C + c] = a;
                }
            /* Tm = (I + A)^-1, unit lower, forward substitution */
            for (int r = 0; r < n; ++r)
                for (int c = 0; c < n; ++c) {
                    double s = (r == c) ? 1.0 : 0.0;
                    for (int j = c; j < r; ++j) s -= A[(size_t)r * C + j] * Tm[(size_t)j * C + c];
                    Tm[(size_t)r * C + c] = (c <= r) ? s : 0.0;
                }
            /* Y = diag(beta) (V - diag(exp gam) K S) */
            for (int r = 0; r < n; ++r) {
                const size_t row = (size_t)(t0 + r) * H + h;
                const double eg = exp(gam[r]);
                for (int j = 0; j < dv; ++j) {
                    double ks = 0.0;
                    for (int i = 0; i < dk; ++i) ks += Kn[(size_t)r * dk + i] * S[(size_t)i * dv + j];
                    Y[(size_t)r * dv + j] = beta[row] * (v[row * dv + j] - eg * ks);
                }
            }
            /* Delta = Tm Y */
            for (int r = 0; r < n; ++r)
                for (int j = 0; j < dv; ++j) {
                    double s = 0.0;
                    for (int c = 0; c <= r; ++c) s += Tm[(size_t)r * C + c] * Y[(size_t)c * dv + j];
                    D[(size_t)r * dv + j] = s;
                }
            /* outputs */
            for (int r = 0; r < n; ++r) {
                const size_t row = (size_t)(t0 + r) * H + h;
                const double eg = exp(gam[r]);
                for (int j = 0; j < dv; ++j) {
                    double qs = 0.0;
                    for (int i = 0; i < dk; ++i) qs += Qn[(size_t)r * dk + i] * S[(size_t)i * dv + j];
                    double o = eg * qs;
                    for (int c = 0; c <= r; ++c) {
                        double s = 0.0, dot = 0.0;
                        for (int jj = c + 1; jj <= r; ++jj) s += GROW(jj);
                        for (int i = 0; i < dk; ++i) dot += Qn[(size_t)r * dk + i] * Kn[(size_t)c * dk + i];
                        o += dot * exp(s) * D[(size_t)c * dv + j];
                    }
                    out[row * dv + j] = o;
                }
            }
            /* state carry */
            {
                double total = 0.0;
                for (int j = 0; j < n; ++j) total += GROW(j);
                const double eg = exp(total);
                for (int i = 0; i < dk; ++i)
                    for (int j = 0; j < dv; ++j) {
                        double s = eg * S[(size_t)i * dv + j];
                        for (int c = 0; c < n; ++c) {
                            double tail = 0.0;
                            for (int jj = c + 1; jj < n; ++jj) tail += GROW(jj);
                            s += exp(tail) * Kn[(size_t)c * dk + i] * D[(size_t)c * dv + j];
                        }
                        Snew[(size_t)i * dv + j] = s;
                    }
                memcpy(S, Snew, sizeof(double) * (size_t)dk * dv);
            }
#undef GROW
        }
        if (final_state)
            memcpy(final_state + (size_t)h * dk * dv, S, sizeof(double) * (size_t)dk * dv);
    }
    free(S); free(Kn); free(Qn); free(gam); free(A); free(Tm); free(Y); free(D); free(Snew);
    return 0;
}

/* Repeat-interleave GQA expansion, qwen.rs:727-738: repeat[i] = i / (Hv/Hk). */
int oracle_delta_scan(const float* q, const float* k, const float* v, const float* g,
                      const float* beta, int T, int Hk, int Hv, int dk, int dv,
                      const float* initial, int capture, float* out, float* captured,
                      float* final_state) {
    if (T < 1 || Hk < 1 || Hv < 1 || Hv % Hk != 0 || dk < 1 || dv < 1) return -1;
    const int rep = Hv / Hk;
    float* qe = (float*)malloc(sizeof(float) * (size_t)T * Hv * dk);
    float* ke = (float*)malloc(sizeof(float) * (size_t)T * Hv * dk);
    for (int t = 0; t < T; ++t)
        for (int h = 0; h < Hv; ++h) {
            memcpy(qe + ((size_t)t * Hv + h) * dk, q + ((size_t)t * Hk + h / rep) * dk, sizeof(float) * dk);
            memcpy(ke + ((size_t)t * Hv + h) * dk, k + ((size_t)t * Hk + h / rep) * dk, sizeof(float) * dk);
        }
    int rc = oracle_delta_recurrence(qe, ke, v, g, beta, T, Hv, dk, dv, initial, capture, out,
                                     captured, final_state);
    free(qe); free(ke);
    return rc;
}

/* ------------------------------------------------------------------ */
/* Pointwise and projection pieces                                     */
/* ------------------------------------------------------------------ */

/* qwen.rs:765-796: y = sum over taps (oldest first) of x[t-delay] * w[c,tap],
 * accumulated from zero, each product rounded before the add. */
void oracle_causal_conv(const float* x, int T, int W, const float* w, int taps, float* y) {
    int t;
#pragma omp parallel for OMP_THREADS schedule(static)
    for (t = 0; t < T; ++t)
        for (int c = 0; c < W; ++c) {
            float acc = 0.0f;
            for (int tap = 0; tap < taps; ++tap) {
                const int delay = taps - 1 - tap;
                if (t >= delay) {
                    const float p = x[(size_t)(t - delay) * W + c] * w[(size_t)c * taps + tap];
                    acc = acc + p;
                }
            }
            y[(size_t)t * W + c] = acc;
        }
}

/* ops.rs:17-32: inverse = 1/sqrt(mean(x^2) + eps); y = (x * inverse) * w. */
void oracle_rms(const float* x, int rows, int width, const float* w, float eps, float* y) {
    const float inv_width = (float)(1.0 / (double)width);
    int r;
#pragma omp parallel for OMP_THREADS schedule(static)
    for (r = 0; r < rows; ++r) {
        const float* xr = x + (size_t)r * width;
        float s = 0.0f;
        for (int i = 0; i < width; ++i) s += xr[i] * xr[i];
        const float root = sqrtf(s * inv_width + eps);
        const float inverse = 1.0f / root;
        for (int i = 0; i < width; ++i) y[(size_t)r * width + i] = (xr[i] * inverse) * w[i];
    }
}

/* Exact-accumulation mode (oracle_set_exact_dots): projection dot products
 * accumulated in f64 and rounded to f32 once.  Not the reference's arithmetic
 * (Candle's f32 GEMM): a yardstick closer to the exact result, against which
 * the f32 restatement and the device path can both be measured. */
static int g_exact_dots = 0;
void oracle_set_exact_dots(int on) { g_exact_dots = on != 0; }

/* y = x W^T.  Eight interleaved partial sums per dot product (a fixed order,
 * so the result does not depend on the thread count). */
static float dot8(const float* a, const float* b, int K) {
    if (g_exact_dots) {
        double d[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        int i = 0;
        for (; i + 8 <= K; i += 8)
            for (int l = 0; l < 8; ++l) d[l] += (double)a[i + l] * (double)b[i + l];
        double s = ((d[0] + d[1]) + (d[2] + d[3])) + ((d[4] + d[5]) + (d[6] + d[7]));
        for (; i < K; ++i) s += (double)a[i] * (double)b[i];
        return (float)s;
    }
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int i = 0;
    for (; i + 8 <= K; i += 8)
        for (int l = 0; l < 8; ++l) acc[l] = acc[l] + a[i + l] * b[i + l];
    float s = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
    for (; i < K; ++i) s = s + a[i] * b[i];
    return s;
}

void oracle_linear(const float* x, int M, int K, const float* w, int N, float* y) {
    /* tile rows x columns so a weight block stays in cache across rows */
    const int NB = 64, MB = 32;
    const int nblocks = (N + NB - 1) / NB, mblocks = (M + MB - 1) / MB;
    int blk;
#pragma omp parallel for OMP_THREADS schedule(dynamic, 1)
    for (blk = 0; blk < nblocks * mblocks; ++blk) {
        const int n0 = (blk % nblocks) * NB, m0 = (blk / nblocks) * MB;
        const int n1 = n0 + NB < N ? n0 + NB : N, m1 = m0 + MB < M ? m0 + MB : M;
        for (int m = m0; m < m1; ++m)
            for (int n = n0; n < n1; ++n)
                y[(size_t)m * N + n] = dot8(x + (size_t)m * K, w + (size_t)n * K, K);
    }
}

static float silu_f(float x) { return x / (1.0f + expf(-x)); }
static float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }

/* ops.rs:62-148: query tiles of 128, key tiles of 256, online softmax in f32. */
int oracle_attention(const float* q, const float* k, const float* v, int heads, int kv_heads,
                     int qn, int kn, int d, int causal, float* out) {
    if (heads < 1 || kv_heads < 1 || heads % kv_heads || d < 1 || qn < 1 || kn < 1 ||
        (causal && qn > kn))
        return -1;
    const float scale = (float)(1.0 / sqrt((double)d));
    const int group = heads / kv_heads;
    const int offset = causal ? kn - qn : 0;
    int task;
    const int qtiles = (qn + 127) / 128;
#pragma omp parallel for OMP_THREADS schedule(dynamic, 1)
    for (task = 0; task < heads * qtiles; ++task) {
        const int h = task / qtiles, qs = (task % qtiles) * 128;
        const int count = qn - qs < 128 ? qn - qs : 128;
        const float* kh = k + (size_t)(h / group) * kn * d;
        const float* vh = v + (size_t)(h / group) * kn * d;
        float* mx = (float*)malloc(sizeof(float) * count);
        float* den = (float*)malloc(sizeof(float) * count);
        float* acc = (float*)calloc((size_t)count * d, sizeof(float));
        float* sc = (float*)malloc(sizeof(float) * 256);
        for (int i = 0; i < count; ++i) { mx[i] = -INFINITY; den[i] = 0.0f; }
        for (int ks = 0; ks < kn; ks += 256) {
            if (causal && ks >= offset + qs + count) break;
            const int keys = kn - ks < 256 ? kn - ks : 256;
            for (int i = 0; i < count; ++i) {
                const float* qr = q + ((size_t)h * qn + qs + i) * d;
                float tile_max = -INFINITY;
                for (int j = 0; j < keys; ++j) {
                    float s = 0.0f;
                    const float* kr = kh + (size_t)(ks + j) * d;
                    for (int e = 0; e < d; ++e) s = s + qr[e] * kr[e];
                    s = s * scale;
                    if (causal && ks + j > offset + qs + i) s = -INFINITY;
                    sc[j] = s;
                    if (s > tile_max) tile_max = s;
                }
                const float nm = mx[i] > tile_max ? mx[i] : tile_max;
                const float rescale = expf(mx[i] - nm);
                float psum = 0.0f;
                float* ar = acc + (size_t)i * d;
                for (int e = 0; e < d; ++e) ar[e] = ar[e] * rescale;
                for (int j = 0; j < keys; ++j) {
                    const float p = expf(sc[j] - nm);
                    psum = psum + p;
                    const float* vr = vh + (size_t)(ks + j) * d;
                    for (int e = 0; e < d; ++e) ar[e] = ar[e] + p * vr[e];
                }
                den[i] = den[i] * rescale + psum;
                mx[i] = nm;
            }
        }
        for (int i = 0; i < count; ++i)
            for (int e = 0; e < d; ++e)
                out[((size_t)h * qn + qs + i) * d + e] = acc[(size_t)i * d + e] / den[i];
        free(mx); free(den); free(acc); free(sc);
    }
    return 0;
}

/* ops.rs:150-185 with text positions [p,p,p] (every mrope axis equal), so the
 * angle of pair i is p * theta^(-2i/dim) (the exponent taken in f64, the
 * product in f32); x*cos + rotate_half(x)*sin on the first dim features. */
void oracle_rotary(float* x, int T, int heads, int width, int dim, double theta, int pos0) {
    const int half = dim / 2;
    float* inv = (float*)malloc(sizeof(float) * (half > 0 ? half : 1));
    for (int i = 0; i < half; ++i) inv[i] = (float)pow(theta, -((double)(2 * i)) / (double)dim);
    float* tmp = (float*)malloc(sizeof(float) * (dim > 0 ? dim : 1));
    for (int t = 0; t < T; ++t) {
        const float p = (float)(pos0 + t);
        for (int h = 0; h < heads; ++h) {
            float* r = x + ((size_t)t * heads + h) * width;
            for (int i = 0; i < dim; ++i) {
                const float ang = p * inv[i % half];
                const float rot = i < half ? -r[i + half] : r[i - half];
                tmp[i] = r[i] * cosf(ang) + rot * sinf(ang);
            }
            memcpy(r, tmp, sizeof(float) * dim);
        }
    }
    free(inv); free(tmp);
}

/* ------------------------------------------------------------------ */
/* Hybrid backbone prefill (qwen.rs:337-426, 451-525, 589-688)          */
/* ------------------------------------------------------------------ */

static void round_if(int mixed, float* x, size_t n) {
    if (mixed) oracle_round_f16(x, n);
}

/* Norm weights: offset norms store w and use 1 + w (normalization.rs:37-46). */
static float* norm_weight(const float* w, int n, int offset, int mixed) {
    float* out = (float*)malloc(sizeof(float) * n);
    for (int i = 0; i < n; ++i) {
        float raw = mixed ? oracle_f16_to_f32(oracle_f32_to_f16(w[i])) : w[i];
        out[i] = offset ? raw + 1.0f : raw;
    }
    return out;
}

/* Projection with the mixed profile's rounding: f16 weights and inputs, f32
 * accumulation, f16 output (neural.metal:7-27). */
static void project(int mixed, const float* x, int M, int K, const float* w, int N, float* y) {
    if (!mixed) {
        oracle_linear(x, M, K, w, N, y);
        return;
    }
    float* wr = (float*)malloc(sizeof(float) * (size_t)N * K);
    memcpy(wr, w, sizeof(float) * (size_t)N * K);
    oracle_round_f16(wr, (size_t)N * K);
    oracle_linear(x, M, K, wr, N, y);
    oracle_round_f16(y, (size_t)M * N);
    free(wr);
}

typedef struct {
    const float* recurrent; /* [Hv,dk,dv] */
    const float* history;   /* [hist,W] */
    int hist;
} delta_in;

/* Delta::forward, qwen.rs:589-688. x [T,H] (already rounded in the mixed profile). */
static void delta_layer(const oracle_backbone* b, const oracle_layer* L, const float* x, int T,
                        const delta_in* init, int capture, float* sav_rec, float* sav_hist,
                        int* sav_hist_rows, float* y) {
    const oracle_config* c = &b->c;
    const int mixed = b->mixed_f16, H = c->hidden;
    const int key = c->lin_k_heads * c->lin_dk, value = c->lin_v_heads * c->lin_dv;
    const int W = 2 * key + value, Hv = c->lin_v_heads, dv = c->lin_dv, taps = c->conv_taps;
    const int hist = init ? init->hist : 0;
    /* projected = qkv(x) -> f32, history prepended (qwen.rs:603-617) */
    float* projected = (float*)malloc(sizeof(float) * (size_t)(hist + T) * W);
    if (hist) memcpy(projected, init->history, sizeof(float) * (size_t)hist * W);
    project(mixed, x, T, H, L->qkv, W, projected + (size_t)hist * W);
    /* conv + silu (qwen.rs:616-618) */
    float* convw = (float*)malloc(sizeof(float) * (size_t)W * taps);
    memcpy(convw, L->conv, sizeof(float) * (size_t)W * taps);
    round_if(mixed, convw, (size_t)W * taps);
    float* conv = (float*)malloc(sizeof(float) * (size_t)(hist + T) * W);
    oracle_causal_conv(projected, hist + T, W, convw, taps, conv);
    float* mixedv = conv + (size_t)hist * W;
    for (size_t i = 0; i < (size_t)T * W; ++i) mixedv[i] = silu_f(mixedv[i]);
    /* g = softplus(a(x) + dt) * -exp(A_log); beta = sigmoid(b(x)) (qwen.rs:619-627) */
    float* a = (float*)malloc(sizeof(float) * (size_t)T * Hv);
    float* bb = (float*)malloc(sizeof(float) * (size_t)T * Hv);
    project(mixed, x, T, H, L->a, Hv, a);
    project(mixed, x, T, H, L->b, Hv, bb);
    float* dt = norm_weight(L->dt, Hv, 0, mixed);
    float* alog = norm_weight(L->a_log, Hv, 0, mixed);
    for (int t = 0; t < T; ++t)
        for (int h = 0; h < Hv; ++h) {
            const float av = a[(size_t)t * Hv + h] + dt[h];
            const float sp = (av > 0.0f ? av : 0.0f) + logf(expf(-fabsf(av)) + 1.0f);
            a[(size_t)t * Hv + h] = sp * -expf(alog[h]);
            bb[(size_t)t * Hv + h] = sigmoid_f(bb[(size_t)t * Hv + h]);
        }
    /* recurrence (qwen.rs:711-756 -> 826-882); q,k,v are views into mixed */
    float* qb = (float*)malloc(sizeof(float) * (size_t)T * key);
    float* kb = (float*)malloc(sizeof(float) * (size_t)T * key);
    float* vb = (float*)malloc(sizeof(float) * (size_t)T * value);
    for (int t = 0; t < T; ++t) {
        memcpy(qb + (size_t)t * key, mixedv + (size_t)t * W, sizeof(float) * key);
        memcpy(kb + (size_t)t * key, mixedv + (size_t)t * W + key, sizeof(float) * key);
        memcpy(vb + (size_t)t * value, mixedv + (size_t)t * W + 2 * key, sizeof(float) * value);
    }
    float* out = (float*)malloc(sizeof(float) * (size_t)T * value);
    oracle_delta_scan(qb, kb, vb, a, bb, T, c->lin_k_heads, Hv, c->lin_dk, dv,
                      init ? init->recurrent : NULL, capture, out, sav_rec, NULL);
    round_if(mixed, out, (size_t)T * value);
    /* gated = rms_w(out) * silu(z) (qwen.rs:671-676) */
    float* z = (float*)malloc(sizeof(float) * (size_t)T * value);
    project(mixed, x, T, H, L->z, value, z);
    float* nw = norm_weight(L->norm, dv, 0, mixed);
    float* gated = (float*)malloc(sizeof(float) * (size_t)T * value);
    oracle_rms(out, T * Hv, dv, nw, c->eps, gated);
    round_if(mixed, gated, (size_t)T * value);
    for (size_t i = 0; i < (size_t)T * value; ++i) gated[i] = gated[i] * silu_f(z[i]);
    round_if(mixed, gated, (size_t)T * value);
    project(mixed, gated, T, value, L->out, H, y);
    /* saved conv history (qwen.rs:677-685) */
    if (capture && sav_hist) {
        const int end = hist + capture;
        const int count = end < taps - 1 ? end : taps - 1;
        memcpy(sav_hist, projected + (size_t)(end - count) * W, sizeof(float) * (size_t)count * W);
        *sav_hist_rows = count;
    }
    free(projected); free(convw); free(conv); free(a); free(bb); free(dt); free(alog);
    free(qb); free(kb); free(vb); free(out); free(z); free(nw); free(gated);
}

/* FullAttention::forward, qwen.rs:451-525.  Gated GQA attention. */
static void attention_layer(const oracle_backbone* b, const oracle_layer* L, const float* x,
                            int T, int pos0, const float* init_k, const float* init_v, int init_n,
                            int capture, float* sav_k, float* sav_v, float* y) {
    const oracle_config* c = &b->c;
    const int mixed = b->mixed_f16, H = c->hidden, d = c->head_dim;
    const int heads = c->heads, kvh = c->kv_heads;
    float* proj = (float*)malloc(sizeof(float) * (size_t)T * heads * 2 * d);
    project(mixed, x, T, H, L->q, heads * 2 * d, proj);
    float* q = (float*)malloc(sizeof(float) * (size_t)T * heads * d);
    float* gate = (float*)malloc(sizeof(float) * (size_t)T * heads * d);
    for (int t = 0; t < T; ++t)
        for (int h = 0; h < heads; ++h) {
            memcpy(q + ((size_t)t * heads + h) * d, proj + ((size_t)t * heads + h) * 2 * d, sizeof(float) * d);
            memcpy(gate + ((size_t)t * heads + h) * d, proj + ((size_t)t * heads + h) * 2 * d + d, sizeof(float) * d);
        }
    float* qnw = norm_weight(L->q_norm, d, 1, mixed);
    float* knw = norm_weight(L->k_norm, d, 1, mixed);
    oracle_rms(q, T * heads, d, qnw, c->eps, q);
    round_if(mixed, q, (size_t)T * heads * d);
    float* kp = (float*)malloc(sizeof(float) * (size_t)T * kvh * d);
    float* vp = (float*)malloc(sizeof(float) * (size_t)T * kvh * d);
    project(mixed, x, T, H, L->k, kvh * d, kp);
    project(mixed, x, T, H, L->v, kvh * d, vp);
    oracle_rms(kp, T * kvh, d, knw, c->eps, kp);
    round_if(mixed, kp, (size_t)T * kvh * d);
    oracle_rotary(q, T, heads, d, c->rotary_dim, c->rope_theta, pos0);
    oracle_rotary(kp, T, kvh, d, c->rotary_dim, c->rope_theta, pos0);
    round_if(mixed, q, (size_t)T * heads * d);
    round_if(mixed, kp, (size_t)T * kvh * d);
    /* to [heads, tokens, d]; prepend cached KV (qwen.rs:486-496) */
    const int kn = init_n + T;
    float* qt = (float*)malloc(sizeof(float) * (size_t)heads * T * d);
    float* kt = (float*)malloc(sizeof(float) * (size_t)kvh * kn * d);
    float* vt = (float*)malloc(sizeof(float) * (size_t)kvh * kn * d);
    for (int h = 0; h < heads; ++h)
        for (int t = 0; t < T; ++t)
            memcpy(qt + ((size_t)h * T + t) * d, q + ((size_t)t * heads + h) * d, sizeof(float) * d);
    for (int h = 0; h < kvh; ++h) {
        if (init_n) {
            memcpy(kt + (size_t)h * kn * d, init_k + (size_t)h * init_n * d, sizeof(float) * (size_t)init_n * d);
            memcpy(vt + (size_t)h * kn * d, init_v + (size_t)h * init_n * d, sizeof(float) * (size_t)init_n * d);
        }
        for (int t = 0; t < T; ++t) {
            memcpy(kt + ((size_t)h * kn + init_n + t) * d, kp + ((size_t)t * kvh + h) * d, sizeof(float) * d);
            memcpy(vt + ((size_t)h * kn + init_n + t) * d, vp + ((size_t)t * kvh + h) * d, sizeof(float) * d);
        }
    }
    if (capture && sav_k) {
        for (int h = 0; h < kvh; ++h) {
            memcpy(sav_k + (size_t)h * capture * d, kt + (size_t)h * kn * d, sizeof(float) * (size_t)capture * d);
            memcpy(sav_v + (size_t)h * capture * d, vt + (size_t)h * kn * d, sizeof(float) * (size_t)capture * d);
        }
    }
    float* att = (float*)malloc(sizeof(float) * (size_t)heads * T * d);
    oracle_attention(qt, kt, vt, heads, kvh, T, kn, d, 1, att);
    round_if(mixed, att, (size_t)heads * T * d);
    /* out = attended^T * sigmoid(gate) -> o_proj (qwen.rs:518-524) */
    float* o = (float*)malloc(sizeof(float) * (size_t)T * heads * d);
    for (int t = 0; t < T; ++t)
        for (int h = 0; h < heads; ++h)
            for (int e = 0; e < d; ++e) {
                float sg = sigmoid_f(gate[((size_t)t * heads + h) * d + e]);
                if (mixed) sg = oracle_f16_to_f32(oracle_f32_to_f16(sg));
                o[((size_t)t * heads + h) * d + e] = att[((size_t)h * T + t) * d + e] * sg;
            }
    round_if(mixed, o, (size_t)T * heads * d);
    project(mixed, o, T, heads * d, L->o, H, y);
    free(proj); free(q); free(gate); free(qnw); free(knw); free(kp); free(vp);
    free(qt); free(kt); free(vt); free(att); free(o);
}

int oracle_backbone_prefill(const oracle_backbone* b, const int* ids, int T,
                            const oracle_prefix* initial, int capture, oracle_prefix* saved,
                            float* hidden_out) {
    const oracle_config* c = &b->c;
    const int H = c->hidden, mixed = b->mixed_f16;
    const int offset = initial ? initial->tokens : 0;
    /* request validation, qwen.rs:345-359 */
    if (T < 1 || offset + T > 4096 || capture < 0 || (capture && capture >= T) ||
        (initial && capture))
        return -1;
    for (int t = 0; t < T; ++t)
        if (ids[t] < 0 || ids[t] >= c->vocab) return -1;
    float* h = (float*)malloc(sizeof(float) * (size_t)T * H);
    for (int t = 0; t < T; ++t)
        memcpy(h + (size_t)t * H, b->embeddings + (size_t)ids[t] * H, sizeof(float) * H);
    round_if(mixed, h, (size_t)T * H);
    float* n = (float*)malloc(sizeof(float) * (size_t)T * H);
    float* y = (float*)malloc(sizeof(float) * (size_t)T * H);
    const int I = c->intermediate;
    float* gbuf = (float*)malloc(sizeof(float) * (size_t)T * I);
    float* ubuf = (float*)malloc(sizeof(float) * (size_t)T * I);
    for (int li = 0; li < c->n_layers; ++li) {
        const oracle_layer* L = &b->layers[li];
        float* inw = norm_weight(L->input_norm, H, 1, mixed);
        float* pnw = norm_weight(L->post_norm, H, 1, mixed);
        oracle_rms(h, T, H, inw, c->eps, n);
        round_if(mixed, n, (size_t)T * H);
        if (L->kind == 0) {
            delta_in din, *dp = NULL;
            if (initial) {
                din.recurrent = initial->recurrent[li];
                din.history = initial->history[li];
                din.hist = initial->history_rows[li];
                dp = &din;
            }
            delta_layer(b, L, n, T, dp, capture, saved && capture ? saved->recurrent[li] : NULL,
                        saved && capture ? saved->history[li] : NULL,
                        saved && capture ? &saved->history_rows[li] : NULL, y);
        } else {
            attention_layer(b, L, n, T, offset, initial ? initial->key[li] : NULL,
                            initial ? initial->value[li] : NULL, offset, capture,
                            saved && capture ? saved->key[li] : NULL,
                            saved && capture ? saved->value[li] : NULL, y);
            if (saved && capture) saved->history_rows[li] = 0;
        }
        for (size_t i = 0; i < (size_t)T * H; ++i) h[i] = h[i] + y[i];
        oracle_rms(h, T, H, pnw, c->eps, n);
        round_if(mixed, n, (size_t)T * H);
        /* down(silu(gate(n)) * up(n)), projection.rs:67-81 */
        project(mixed, n, T, H, L->gate, I, gbuf);
        project(mixed, n, T, H, L->up, I, ubuf);
        for (size_t i = 0; i < (size_t)T * I; ++i) {
            float s = silu_f(gbuf[i]);
            if (mixed) s = oracle_f16_to_f32(oracle_f32_to_f16(s));
            gbuf[i] = s * ubuf[i];
        }
        round_if(mixed, gbuf, (size_t)T * I);
        project(mixed, gbuf, T, I, L->down, H, y);
        for (size_t i = 0; i < (size_t)T * H; ++i) h[i] = h[i] + y[i];
        free(inw); free(pnw);
    }
    float* fw = norm_weight(b->final_norm, H, 1, mixed);
    float* hidden = hidden_out + (size_t)offset * H;
    oracle_rms(h, T, H, fw, c->eps, hidden);
    if (initial) memcpy(hidden_out, initial->hidden, sizeof(float) * (size_t)offset * H);
    if (saved && capture) {
        saved->tokens = capture;
        memcpy(saved->hidden, hidden, sizeof(float) * (size_t)capture * H);
    }
    free(fw); free(h); free(n); free(y); free(gbuf); free(ubuf);
    return 0;
}

/*
 * clef_oracle.h -- CPU restatement of the clef-rs hybrid-backbone prefill path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker and the CPU
 * baseline.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it, and only to check or time the HIP path -- never as the
 * product.  The product library (libclef_hip.so) never links or calls it.
 *
 * Every function restates the reference's CPU F32 algorithm and cites the
 * file:line it follows (paths relative to the clef-rs repository root):
 *   crates/core/src/models/qwen.rs   (layer loop, DeltaNet mixer, conv, recurrence,
 *                                     gated attention layer)
 *   crates/core/src/models/ops.rs    (RMSNorm, tiled causal attention, rotary)
 *   crates/core/src/models/chunk.metal + transformers' chunk_gated_delta_rule
 *                                    (chunkwise WY/UT algebra, used only as a
 *                                     cross-check of the per-token form)
 *
 * Pinning (what checks each function; see tests/test_oracle.py):
 *   oracle_backbone_prefill ... golden hidden states of the reference's
 *       synthetic backbone fixture (3 DeltaNet + 1 gated attention layer,
 *       T=20), tolerance 1e-5 + 1e-4|e| as the reference test uses.
 *   oracle_delta_recurrence ... f64 brute force, closed forms (T=1, beta=0,
 *       g=-inf token independence, orthonormal exact writes), the chunked f64
 *       form, split/resume invariance, and the fixture above.
 *   oracle_linear / rms / conv / attention / rotary ... the fixture above
 *       plus textbook closed forms (dense softmax attention, f64 dot products).
 * Parity unpinned: bit-level agreement with Candle's CPU kernels (no
 * reference test pins that; only tolerances are pinned).
 */
#ifndef CLEF_ORACLE_H
#define CLEF_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- f16 rounding helpers (IEEE binary16, round-to-nearest-even) ---- */
uint16_t oracle_f32_to_f16(float x);
float oracle_f16_to_f32(uint16_t h);
void oracle_round_f16(float* x, size_t n);

/* ---- gated delta rule ----
 * Per-token recurrence, qwen.rs:826-882.  q,k,v are raw (pre-norm) and already
 * head-expanded: q,k [T,H,dk], v [T,H,dv], g,beta [T,H] (g is log-decay).
 * initial [H,dk,dv] or NULL; capture in 1..T or 0 (none).
 * out [T,H,dv]; captured [H,dk,dv] (state after token `capture`), may be NULL;
 * final_state [H,dk,dv] (state after the last token), may be NULL.
 * Returns 0, or -1 on invalid dimensions (checked before any work). */
int oracle_delta_recurrence(const float* q, const float* k, const float* v, const float* g,
                            const float* beta, int T, int H, int dk, int dv,
                            const float* initial, int capture, float* out, float* captured,
                            float* final_state);
/* Same recurrence in double precision (brute-force golden). */
int oracle_delta_recurrence_f64(const double* q, const double* k, const double* v,
                                const double* g, const double* beta, int T, int H, int dk,
                                int dv, const double* initial, double* out, double* final_state);
/* Chunkwise WY/UT form in double precision (chunk.metal:10-164 algebra). */
int oracle_delta_chunked_f64(const double* q, const double* k, const double* v, const double* g,
                             const double* beta, int T, int H, int dk, int dv, int chunk,
                             const double* initial, double* out, double* final_state);
/* GQA wrapper, qwen.rs:711-756: q,k [T,Hk,dk], v [T,Hv,dv]; v-head i reads
 * k-head i/(Hv/Hk) (repeat-interleave). */
int oracle_delta_scan(const float* q, const float* k, const float* v, const float* g,
                      const float* beta, int T, int Hk, int Hv, int dk, int dv,
                      const float* initial, int capture, float* out, float* captured,
                      float* final_state);

/* ---- pointwise / projection pieces ---- */
/* Depthwise causal conv, oldest->newest taps, qwen.rs:765-796. w [W,taps]. */
void oracle_causal_conv(const float* x, int T, int W, const float* w, int taps, float* y);
/* RMSNorm, ops.rs:17-32: y = (x * 1/sqrt(mean(x^2)+eps)) * w (w already offset). */
void oracle_rms(const float* x, int rows, int width, const float* w, float eps, float* y);
/* y[M,N] = x[M,K] . W[N,K]^T, f32 accumulation. */
void oracle_linear(const float* x, int M, int K, const float* w, int N, float* y);
/* Tiled causal/non-causal attention with online softmax, ops.rs:62-148.
 * q [heads,qn,d], k,v [kv_heads,kn,d] -> out [heads,qn,d]. */
int oracle_attention(const float* q, const float* k, const float* v, int heads, int kv_heads,
                     int qn, int kn, int d, int causal, float* out);
/* Rotary on the first `dim` features, rotate-half convention, ops.rs:150-185.
 * x [T,heads,width] in place; position of row t is pos0 + t. */
void oracle_rotary(float* x, int T, int heads, int width, int dim, double theta, int pos0);

/* ---- hybrid backbone (qwen.rs:365-426) ---- */
typedef struct {
    int hidden, intermediate, vocab;
    int heads, kv_heads, head_dim, rotary_dim;         /* gated full attention */
    int lin_k_heads, lin_v_heads, lin_dk, lin_dv, conv_taps;
    int n_layers;
    float eps;
    double rope_theta;
} oracle_config;

/* Raw weights as stored in the checkpoint (norm offsets applied inside). */
typedef struct {
    int kind; /* 0 = linear_attention (DeltaNet), 1 = full_attention */
    const float *input_norm, *post_norm, *gate, *up, *down;
    /* DeltaNet: qkv [2Hk*dk+Hv*dv, H], z [Hv*dv,H], a,b [Hv,H], out [H,Hv*dv],
     * conv [W,taps], dt [Hv], a_log [Hv], norm [dv] */
    const float *qkv, *z, *a, *b, *out, *conv, *dt, *a_log, *norm;
    /* attention: q [2*heads*d,H], k,v [kvh*d,H], o [H,heads*d], q_norm,k_norm [d] */
    const float *q, *k, *v, *o, *q_norm, *k_norm;
} oracle_layer;

typedef struct {
    oracle_config c;
    const float* embeddings; /* [vocab, H] */
    const float* final_norm; /* [H] raw */
    const oracle_layer* layers;
    int mixed_f16; /* 1: emulate the mixed-F16 profile's half-rounding points */
} oracle_backbone;

/* Per-layer continuation state (PrefixState, qwen.rs:153-191).  Buffers are
 * caller-owned, sized by oracle_prefix_sizes. */
typedef struct {
    int tokens;            /* boundary token count */
    float* hidden;         /* [tokens, H] */
    float** recurrent;     /* per DeltaNet layer [Hv,dk,dv] (NULL entries for attention) */
    float** history;       /* per DeltaNet layer [hist_rows, W] */
    int* history_rows;     /* per layer */
    float** key;           /* per attention layer [kvh, tokens, d] */
    float** value;         /* per attention layer [kvh, tokens, d] */
} oracle_prefix;

/* Prefill (qwen.rs:337-426).  ids [T]; hidden_out [(offset+T), H] where
 * offset = initial ? initial->tokens : 0.  capture in 1..T-1 or 0.
 * Returns 0, or -1 on invalid request. */
int oracle_backbone_prefill(const oracle_backbone* b, const int* ids, int T,
                            const oracle_prefix* initial, int capture, oracle_prefix* saved,
                            float* hidden_out);

/* Threads used by the OpenMP regions (0 = runtime default). */
void oracle_set_threads(int n);
/* f64-accumulated projection dot products (a yardstick, not the reference's arithmetic). */
void oracle_set_exact_dots(int on);
int oracle_get_threads(void);

#ifdef __cplusplus
}
#endif
#endif

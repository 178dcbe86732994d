/*
 * clef_hip.h -- C ABI of the MI355X (gfx950) hybrid-backbone prefill path.
 *
 * Each entry point replaces one device custom op of clef-rs's Metal backend
 * (paths relative to the clef-rs repository root) and keeps its semantics:
 * the same shapes, the same op contract, validation before any launch.
 *
 * Conventions
 *  - Buffers are device pointers owned by the caller; the library allocates
 *    no persistent memory.  Scratch space is passed in as `workspace`.
 *  - Every call is asynchronous on `stream` (a hipStream_t; NULL = the null
 *    stream) and never synchronizes the host.
 *  - Return value: 0 on success; < 0 validation error (nothing was launched);
 *    > 0 a HIP error code from the launch.  clef_hip_last_error() returns the
 *    message of the calling thread's last failure.
 *  - Tensors are row-major.  "Token stride" arguments give the distance in
 *    elements between consecutive tokens (rows) so that views into a packed
 *    projection output can be passed without a copy; 0 means contiguous.
 *  - dtype codes: CLEF_F32 = 0, CLEF_F16 = 1 (IEEE binary16).
 */
#ifndef CLEF_HIP_H
#define CLEF_HIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { CLEF_F32 = 0, CLEF_F16 = 1 };
/* Scan arithmetic profile.  STRICT: f32 operands on f32 MFMA (parity with the
 * CPU F32 path at rtol 1e-4 / atol 1e-5).  MIXED: f16 operands on f16 MFMA
 * with f32 accumulation and an f32 state (rtol 2e-2). */
enum { CLEF_SCAN_STRICT = 0, CLEF_SCAN_MIXED = 1 };

const char* clef_hip_last_error(void);
int clef_hip_abi_version(void);

/* ---------------------------------------------------------------------- */
/* Gated DeltaNet scan                                                     */
/* ---------------------------------------------------------------------- */
/*
 * Replaces DeltaKernel::{forward, prepared_prefill, prefill} and the
 * "clef-fused-delta" / "clef-cached-delta" custom ops
 * (crates/core/src/models/metal.rs:161-278, 291-413), whose CPU definition is
 * delta_recurrence_prefill (crates/core/src/models/qwen.rs:826-882):
 *   q <- l2(q)/sqrt(dk), k <- l2(k), l2(x) = x/sqrt(sum x^2 + 1e-6)
 *   per token: S <- S*exp(g); d = (v - S^T k)*beta; S <- S + k d^T; o = S^T q
 * with v-head i reading k-head i/(Hv/Hk) (repeat-interleave, qwen.rs:727-738).
 *
 * q, k: [T, Hk, dk] (token strides sqk, dtype_qkv); v: [T, Hv, dv] (token
 * stride sv, dtype_qkv); g (log-decay), beta: [T, Hv] (token stride sgb,
 * dtype_gb).  out: [T, Hv, dv] (token stride so, dtype_out).
 * initial: [Hv, dk, dv] f32 or NULL (zero state).  capture in 1..T writes the
 * state after token `capture` to captured [Hv, dk, dv]; 0 = none.
 * final_state [Hv, dk, dv] f32 or NULL receives the state after token T.
 * Limits: 1 <= T <= 1048576; 1 <= Hk <= Hv <= 256; Hv % Hk == 0;
 * 1 <= dk <= 128; 1 <= dv <= 128; chunk == 64.
 */
size_t clef_delta_scan_workspace(int T, int Hk, int Hv, int dk, int dv, int chunk, int precision);
int clef_delta_scan(const void* q, const void* k, const void* v, int64_t sqk, int64_t sv,
                    int dtype_qkv, const void* g, const void* beta, int64_t sgb, int dtype_gb,
                    int T, int Hk, int Hv, int dk, int dv, int chunk, int precision,
                    const float* initial, int capture, void* out, int64_t so, int dtype_out,
                    float* captured, float* final_state, void* workspace, size_t workspace_bytes,
                    void* stream);

/*
 * clef_delta_scan without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops or
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * scan's scratch is a file-scope device array of CLEF_SCAN_SCRATCH_BYTES
 * (96 MiB) in this library, one per GPU: the runtime reserves it on each GPU
 * when it loads the library's device code there, whether or not this entry
 * point is ever called, and holds it until the process ends (its address is
 * looked up once per device, at the first call with that device current;
 * the stream must belong to the current device).  A shape whose
 * clef_delta_scan_workspace exceeds it is rejected before any launch (the
 * full layer shape T = 4096, Hk = 16, Hv = 32, dk = dv = 128 needs 50.5 MiB in
 * the mixed profile and 99 MiB, which is refused, in the strict one).
 * Arguments and results as clef_delta_scan.  Every call
 * on a GPU uses that GPU's one array: calls that overlap in time on one GPU
 * (other streams, other threads) race, and the caller must serialize them.
 */
#define CLEF_SCAN_SCRATCH_BYTES ((size_t)96 << 20)
int clef_delta_scan_noalloc(const void* q, const void* k, const void* v, int64_t sqk, int64_t sv,
                            int dtype_qkv, const void* g, const void* beta, int64_t sgb, int dtype_gb,
                            int T, int Hk, int Hv, int dk, int dv, int chunk, int precision,
                            const float* initial, int capture, void* out, int64_t so, int dtype_out,
                            float* captured, float* final_state, void* stream);

/*
 * Ragged batch of nseq independent sequences packed along the token axis
 * (T tokens in total; sequence s is tokens cu_seqlens[s] .. cu_seqlens[s+1]-1,
 * cu_seqlens a device int32 array of nseq + 1 non-decreasing offsets in
 * [0, T]; see clef_ragged_plan for other tables).  Each sequence runs the
 * recurrence above from its own initial
 * state: initial + s * initial_stride floats ([Hv, dk, dv] f32; stride 0 =
 * one state shared by all, NULL = zero states); final_states, if not NULL,
 * receives [nseq, Hv, dk, dv].  Layouts, dtypes and limits as above, with
 * 1 <= nseq <= 4096; no capture.  No counterpart in the reference, which runs
 * one request per CachedDelta call (metal.rs:340-413): this batches those
 * calls (prefix hits resume every request from the same PrefixState).
 */
size_t clef_delta_scan_varlen_workspace(int T, int nseq, int Hk, int Hv, int dk, int dv, int chunk,
                                        int precision);
/*
 * Ragged batches and malformed offsets: the scan (clef_delta_scan_varlen)
 * and attention (clef_attention_gated_varlen) first make the offsets
 * monotone, R[j] = max over i <= j of cu_seqlens[i] clamped to [0, T], and
 * sequence s is then tokens R[s] .. R[s+1]-1 (R equals cu_seqlens for a
 * valid table).  The conv (clef_conv_silu_varlen) and the q/k norm + rotary
 * (clef_qk_norm_rotary_varlen) find a token t's sequence by binary search
 * over cu_seqlens as given and clamp that sequence's first token into
 * [0, t]; for a valid table this is the same partition.  So an offset table
 * the host cannot inspect (it is device memory) never takes a kernel outside
 * its buffers: a malformed one gives unspecified values, never an access
 * out of bounds.  clef_ragged_plan evaluates the scan's and attention's
 * tables on the host, with the
 * device kernels' code: cu_seqlens in host memory; unit 64 (the scan's
 * chunks) or 128 (attention's query tiles); spans receives R ([nseq + 1]);
 * table, if not NULL, receives the units (scan: {first token, tokens} per
 * chunk; attention: {sequence, tile} in launch order), table_entries >=
 * ceil(T / unit) + nseq.  Returns the unit count (at most that bound) or < 0.
 * No counterpart in the reference (one request per call there).
 */
int clef_ragged_plan(const int32_t* cu_seqlens, int nseq, int T, int unit, int32_t* spans, int32_t* table,
                     size_t table_entries);
int clef_delta_scan_varlen(const void* q, const void* k, const void* v, int64_t sqk, int64_t sv,
                           int dtype_qkv, const void* g, const void* beta, int64_t sgb, int dtype_gb,
                           const int32_t* cu_seqlens, int nseq, int T, int Hk, int Hv, int dk, int dv,
                           int chunk, int precision, const float* initial, int64_t initial_stride,
                           void* out, int64_t so, int dtype_out, float* final_states, void* workspace,
                           size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------- */
/* Projections                                                             */
/* ---------------------------------------------------------------------- */
/*
 * y[M,N] = x[M,K] . W[N,K]^T  (W row-major [N,K], the checkpoint layout).
 * Replaces GemmKernel::forward / "clef-metal4-gemm" (neural.rs:50-55,
 * 151-173; neural.metal:72-97) and candle_nn::Linear (projection.rs:82-95).
 * dtype_in CLEF_F16: f16 operands on f16 MFMA, f32 accumulation;
 * CLEF_F32: f32 operands on f32 MFMA.  x and W share dtype_in.
 * epilogue: CLEF_EPI_STORE writes y in dtype_out (f16 output is rounded once
 * from the f32 accumulator, as neural.metal:23-26);
 * CLEF_EPI_RESIDUAL adds the (dtype_out-rounded) product into an f32 residual
 * y (h += to_f32(round(x W^T)), qwen.rs:399-410).
 * Leading dimensions ldx, ldw, ldy in elements (0 = K, K, N).
 */
enum { CLEF_EPI_STORE = 0, CLEF_EPI_RESIDUAL = 1 };
int clef_gemm(const void* x, int64_t ldx, const void* w, int64_t ldw, void* y, int64_t ldy,
              int M, int N, int K, int dtype_in, int dtype_out, int epilogue, void* stream);
/*
 * y[M,N] = silu(x Wg^T) * (x Wu^T).  Replaces GemmKernel::gated /
 * "clef-metal4-gated" (neural.rs:56-58; neural.metal:29-44, 99-125) and
 * Projection::gated_forward (projection.rs:67-81).  In f16 the gate, its silu,
 * the up product and the result are each rounded to half, as the reference
 * kernel does.
 */
int clef_gemm_swiglu(const void* x, int64_t ldx, const void* wg, const void* wu, int64_t ldw,
                     void* y, int64_t ldy, int M, int N, int K, int dtype, void* stream);

/* ---------------------------------------------------------------------- */
/* Pointwise pieces around the scan                                        */
/* ---------------------------------------------------------------------- */
/*
 * RMSNorm y = (x * 1/sqrt(mean(x^2)+eps)) * w, rows of `width`.
 * Replaces Rms::forward / "clef-rms" (normalization.rs:62-74; ops.rs:17-32;
 * pointwise.metal:7-43).  w is f32 and already includes any (1+w) offset.
 * x token stride ldx, y token stride ldy (0 = width).
 */
int clef_rms_norm(const void* x, int64_t ldx, int dtype_in, const float* w, void* y, int64_t ldy,
                  int dtype_out, int rows, int width, float eps, void* stream);
/*
 * Depthwise causal conv (taps oldest->newest, zero padded) followed by SiLU,
 * over `history_rows` cached rows followed by T new rows.  Replaces
 * causal_convolution + silu (qwen.rs:609-618, 765-796) and "clef-conv"
 * (pointwise.metal:46-65).  x: [T, W] (stride ldx, dtype_in); history:
 * [history_rows, W] f32 or NULL; w: [W, taps] f32; y: [T, W] (stride ldy,
 * dtype_out).  taps <= 8, history_rows <= taps - 1.
 */
int clef_conv_silu(const void* x, int64_t ldx, int dtype_in, const float* history,
                   int history_rows, const float* w, int taps, void* y, int64_t ldy, int dtype_out,
                   int T, int W, void* stream);
/*
 * Ragged batch of the same conv: sequence s is tokens cu_seqlens[s] ..
 * cu_seqlens[s+1]-1 (device int32, nseq + 1 offsets) and its history rows
 * start at history + s * history_stride floats (stride 0: one history, e.g. a
 * shared prefix).  taps <= 8.  No counterpart in the reference (one request
 * per call there).
 */
int clef_conv_silu_varlen(const void* x, int64_t ldx, int dtype_in, const float* history,
                          int history_rows, int64_t history_stride, const int32_t* cu_seqlens, int nseq,
                          const float* w, int taps, void* y, int64_t ldy, int dtype_out, int T, int W,
                          void* stream);
/*
 * Decay and write strength from the a/b projections (qwen.rs:619-627):
 * g = softplus(a + dt) * -exp(A_log) (stable softplus), beta = sigmoid(b).
 * a, b: [T, Hv] (token strides lda, ldb, dtype_in); dt, a_log: [Hv] f32;
 * g, beta: [T, Hv] f32 contiguous.
 */
int clef_delta_gates(const void* a, int64_t lda, const void* b, int64_t ldb, int dtype_in,
                     const float* dt, const float* a_log, float* g, float* beta, int T, int Hv,
                     void* stream);
/*
 * The a/b projections and the gates in one launch (f16 operands): [a | b] =
 * x . w_ab^T with f32 accumulation, each value rounded to f16 as the
 * reference's separate in_proj_a / in_proj_b projections store it
 * (qwen.rs:612-623), then g and beta as clef_delta_gates.  w_ab: [2 Hv, K]
 * (row stride ldw), rows 0..Hv-1 in_proj_a and Hv..2Hv-1 in_proj_b, packed
 * once by clef_delta_gates_pack into a device buffer of
 * clef_delta_gates_pack_bytes(K, Hv) bytes (MFMA fragment order; 16-byte
 * aligned).  x: [T, K] (row stride ldx); g, beta: [T, Hv] f32.  Hv in
 * {16, 32, 64}, K a multiple of 256 up to 4096, rows 16-byte aligned.  Lets
 * the in-projection GEMM cover [qkv | z] only (a whole number of 256-column
 * tiles).
 */
size_t clef_delta_gates_pack_bytes(int K, int Hv);
int clef_delta_gates_pack(const void* w_ab, int64_t ldw, int K, int Hv, int dtype, void* packed, void* stream);
int clef_delta_gates_proj(const void* x, int64_t ldx, const void* packed, int K, int dtype, const float* dt,
                          const float* a_log, float* g, float* beta, int T, int Hv, void* stream);
/*
 * The unfused SwiGLU product (the gated_forward fallback of projection.rs:
 * 67-81: silu(gate) * up on separate projections): y[i] = silu(gate[i]) *
 * up[i] over n elements of dtype (all three arrays).  f16: the half roundings
 * of neural.metal:35-42 with the same SiLU as clef_gemm_swiglu's f16
 * epilogue, so clef_gemm_swiglu equals clef_gemm + clef_gemm + this bit for
 * bit (the reference's fused-vs-unfused rule, neural.rs:484-492).
 */
int clef_silu_mul(const void* gate, const void* up, void* y, int64_t n, int dtype, void* stream);
/*
 * Gated output norm, qwen.rs:671-676: per token and v-head row of `width`,
 * o is rounded to dtype_out (the scan output cast to the activation dtype),
 * RMS-normalised in f32 with w (no offset), rounded to dtype_out, multiplied
 * by silu(z) in f32 and rounded to dtype_out.  o: [T, Hv, width] contiguous
 * in dtype_o (a scan that already wrote o in f16 gives the same values as
 * rounding its f32 output here); z: [T, Hv, width] with token stride ldz
 * (dtype_z); y: [T, Hv*width] contiguous.
 */
int clef_gated_rms_silu(const void* o, int dtype_o, const void* z, int64_t ldz, int dtype_z, const float* w,
                        void* y, int dtype_out, int T, int Hv, int width, float eps, void* stream);

/* ---------------------------------------------------------------------- */
/* Gated full-attention layer pieces (qwen.rs:451-525; ops.rs:62-188)      */
/* ---------------------------------------------------------------------- */
/*
 * Per-head RMSNorm then rotary, for the attention q and k (qwen.rs:437-470;
 * ops.rs:17-32, 150-185).  x: [T, heads, *] with token stride ldx and head
 * stride hs (the q projection interleaves [q | gate] per head, so hs = 2d);
 * w: [d] f32 norm weights, already offset (1 + w).  The norm output is
 * rounded to dtype_out, rotated on the first rot_dim features (rotate-half;
 * angle (pos0 + t) * theta^(-2i/rot_dim), the exponent taken in f64) and
 * rounded again.  y is head-major [heads, ldy_tok, d]: row (h, dst_offset + t).
 */
int clef_qk_norm_rotary(const void* x, int64_t ldx, int64_t hs, int dtype_in, const float* w,
                        void* y, int64_t ldy_tok, int dtype_out, int T, int heads, int d,
                        int rot_dim, double theta, int pos0, int dst_offset, float eps,
                        void* stream);
/* Ragged batch: token t of sequence s takes position pos0 + (t - cu_seqlens[s])
 * (cu_seqlens: device int32, nseq + 1 offsets); rows stay packed. */
int clef_qk_norm_rotary_varlen(const void* x, int64_t ldx, int64_t hs, int dtype_in, const float* w,
                               void* y, int64_t ldy_tok, int dtype_out, int T, int heads, int d,
                               int rot_dim, double theta, int pos0, const int32_t* cu_seqlens, int nseq,
                               int dst_offset, float eps, void* stream);
/*
 * Value layout for attention: x [T, heads, d] (token stride ldx, head stride
 * d) -> y transposed per head, [heads, d, ldy_tok] with token (dst_offset + t)
 * contiguous, so that P.V reads 16-byte runs of consecutive keys.
 */
int clef_values_transposed(const void* x, int64_t ldx, int dtype_in, void* y, int64_t ldy_tok,
                           int dtype_out, int T, int heads, int d, int dst_offset, void* stream);
/*
 * Causal GQA attention with online softmax (bottom-right aligned mask when
 * kn > qn) and sigmoid output gate:
 *   y[t, h*d + e] = attn(q,k,v)[h, t, e] * sigmoid(gate[t, h, e])
 * Replaces ops::attention + the gate of qwen.rs:511-524 and the
 * "clef-f32-flash-attention" op (metal.rs:528-633).
 * q [heads, ldq_tok, d] (rows 0..qn-1), k [kv_heads, ldk_tok, d],
 * vt [kv_heads, d, ldv_tok] (from clef_values_transposed); gate token stride
 * ldg and head stride hsg; y [qn, heads*d] token stride ldy.  dtype is the
 * operand dtype of q/k/v/gate (f16: f16 MFMA, f32: f32 MFMA), accumulation
 * and softmax in f32; y in dtype (the product of the rounded attention and
 * the rounded gate, as the reference's mixed profile does).  d in {64, 128,
 * 256}; heads % kv_heads == 0; qn <= kn.
 */
int clef_attention_gated(const void* q, int64_t ldq_tok, const void* k, int64_t ldk_tok,
                         const void* vt, int64_t ldv_tok, int dtype, int heads, int kv_heads,
                         int qn, int kn, int d, const void* gate, int64_t ldg, int64_t hsg,
                         void* y, int64_t ldy, void* stream);
/*
 * clef_attention_gated with the query RMS norm and rotary of qwen.rs:459-468
 * (as clef_qk_norm_rotary computes them, bit for bit) folded into the
 * attention core's query loads: row t of head h is read raw, f16, at
 * q_raw + t * ldq_row + h * hsq, normalised with q_norm (d weights, eps) and
 * rotated on its first 64 features by rot_tab row t (the cos, sin pairs of
 * clef_rotary_table for the same positions).  One f16 sequence, d = 256,
 * rotary width 64, 16-byte aligned rows, weights and table.  No counterpart
 * in the reference (there the norm and rotary are their own passes); it
 * saves the query pass of clef_qk_norm_rotary and its [heads, qn, d] copy.
 */
int clef_attention_gated_qnorm(const void* q_raw, int64_t ldq_row, int64_t hsq, const float* q_norm, float eps,
                               const float* rot_tab, const void* k, int64_t ldk_tok, const void* vt,
                               int64_t ldv_tok, int heads, int kv_heads, int qn, int kn, int d, const void* gate,
                               int64_t ldg, int64_t hsg, void* y, int64_t ldy, void* stream);
/*
 * The rotary (cos, sin) pairs of positions pos0 .. pos0 + T - 1, as
 * clef_qk_norm_rotary forms them (ops.rs:165-188: the angle rounded once in
 * f32, then cos and sin), written as out[t][i] = {cos, sin} of frequency i
 * < rot_dim / 2 (float pairs, [T][rot_dim / 2][2]).  The table of
 * clef_attention_gated_qnorm.
 */
int clef_rotary_table(int T, int rot_dim, double theta, int pos0, float* out, void* stream);
/*
 * Ragged batch (mixed profile, dtype f16): sequence s owns packed rows
 * cu_seqlens[s] .. cu_seqlens[s+1]-1 (device int32, nseq + 1 offsets in
 * [0, T]) of q [heads, ldq_tok, d], k [kv_heads, ldk_tok, d], vt
 * [kv_heads, d, ldv_tok], gate and y, and its queries see np prefix keys
 * (prefix_k [kv_heads, ldpk_tok, d], prefix_vt [kv_heads, d, ldpv_tok]; all
 * visible, np % 8 == 0, 0 with NULL buffers) before its own, causally: each
 * sequence equals clef_attention_gated over [prefix; own] keys.  The
 * workspace (clef_attention_varlen_workspace) holds the launch tables.  No
 * counterpart in the reference (one request per flash-attention call there).
 */
size_t clef_attention_varlen_workspace(int T, int nseq);
int clef_attention_gated_varlen(const void* q, int64_t ldq_tok, const void* k, int64_t ldk_tok,
                                const void* vt, int64_t ldv_tok, const int32_t* cu_seqlens, int nseq, int T,
                                const void* prefix_k, int64_t ldpk_tok, const void* prefix_vt,
                                int64_t ldpv_tok, int np, int dtype, int heads, int kv_heads, int d,
                                const void* gate, int64_t ldg, int64_t hsg, void* y, int64_t ldy,
                                void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------- */
/* Embedding gather and pooled head                                         */
/* ---------------------------------------------------------------------- */
/* h[t, :] = f32(table[ids[t], :]); ids are int32 and must be < vocab. */
int clef_embed(const int32_t* ids, int T, const void* table, int dtype, int vocab, int H, float* h,
               void* stream);
/* logits[j] = sum_k x[row, k] * W[j, k], f32 (last-token pooled head). */
int clef_head_logits(const float* x, int H, const float* w, int n_logits, float* logits,
                     void* stream);

/* ---------------------------------------------------------------------- */
/* Hybrid backbone prefill (host orchestration over the kernels above)     */
/* ---------------------------------------------------------------------- */
/*
 * Replaces Backbone::{load, prefill, forward} (crates/core/src/models/qwen.rs:
 * 193-426) with the DeltaNet mixer Delta::forward (:589-688) and the gated
 * attention layer FullAttention::forward (:451-525).  Layer kinds: 0 =
 * linear_attention (DeltaNet), 1 = full_attention.
 *
 * Profiles: CLEF_PROFILE_F32 runs every projection on f32 MFMA and the strict
 * scan (the reference's CPU/Metal F32 profile); CLEF_PROFILE_MIXED_F16 runs
 * f16 projections with f32 accumulation and the reference's half rounding
 * points, an f32 residual stream, and the scan in `scan_precision`.
 */
enum { CLEF_PROFILE_F32 = 0, CLEF_PROFILE_MIXED_F16 = 1 };

typedef struct {
    int hidden, intermediate, vocab;
    int heads, kv_heads, head_dim, rotary_dim;
    int lin_k_heads, lin_v_heads, lin_dk, lin_dv, conv_taps;
    int n_layers;
    float eps;
    double rope_theta;
    int profile;        /* CLEF_PROFILE_* */
    int scan_precision; /* CLEF_SCAN_* */
    int max_tokens;     /* prefix + new tokens per prefill (reference: 4096) */
} clef_backbone_config;

/* Device pointers to one layer's checkpoint tensors.  Matrices ([out, in],
 * row-major) are in the profile dtype (f16 for MIXED_F16, f32 for F32);
 * vectors and the conv kernel are f32 and raw (the (1+w) norm offsets are
 * applied at create, normalization.rs:37-46).  Unused fields may be NULL. */
typedef struct {
    int kind;
    const void *input_norm, *post_norm;          /* [H] f32 */
    const void *gate, *up, *down;                /* [I,H], [I,H], [H,I] */
    const void *qkv, *z, *a, *b, *out;           /* DeltaNet projections */
    const void *conv, *dt, *a_log, *norm;        /* [W,taps], [Hv], [Hv], [dv] f32 */
    const void *q, *k, *v, *o;                   /* attention projections */
    const void *q_norm, *k_norm;                 /* [d] f32 */
} clef_layer_weights;

typedef struct clef_backbone clef_backbone;

/* Copies what it must (fused in-projections, offset norms) into memory the
 * backbone owns until clef_backbone_destroy; the MLP and output matrices and
 * the embedding table are referenced in place and must outlive it. */
int clef_backbone_create(const clef_backbone_config* config, const clef_layer_weights* layers,
                         const void* embeddings, const void* final_norm, clef_backbone** out);
void clef_backbone_destroy(clef_backbone* b);
/* Workspace for a prefill of T new tokens after `prefix_tokens` cached ones. */
size_t clef_backbone_workspace(const clef_backbone* b, int T, int prefix_tokens);
/* Bytes of a prefix state (PrefixState, qwen.rs:153-191) at `tokens`. */
size_t clef_backbone_prefix_bytes(const clef_backbone* b, int tokens);
/*
 * ids: host int32 [T], each < vocab.  initial: a prefix state buffer written
 * by an earlier capture (initial_tokens of them), or NULL; initial_bytes is
 * its size and must equal clef_backbone_prefix_bytes(b, initial_tokens), so a
 * state captured by a backbone of another shape (the reference's layer-count
 * check, qwen.rs:355) or passed with the wrong token count is rejected before
 * any launch.  capture in 1..T-1 writes the state after `capture` tokens into
 * `saved` (saved_bytes >= clef_backbone_prefix_bytes(b, capture)); initial
 * and capture are exclusive (qwen.rs:345-359).  hidden: f32
 * [(initial_tokens + T), H], the final-normed hidden states, prefix rows
 * included.
 */
int clef_backbone_prefill(clef_backbone* b, const int32_t* ids, int T, const void* initial,
                          int initial_tokens, size_t initial_bytes, int capture, void* saved,
                          size_t saved_bytes, float* hidden, void* workspace, size_t workspace_bytes,
                          void* stream);
/*
 * Ragged batch of requests resumed from one shared prefix state (a prefix
 * cache hit for each, prefix_cache.rs:135-177): ids is the host int32 packed
 * token stream, cu_seqlens the host int32 offsets (cu_seqlens[0] = 0, each
 * sequence 1..max_tokens - initial_tokens long, at most 4096 sequences and
 * 2^20 tokens; initial_bytes as for clef_backbone_prefill).  hidden: f32
 * [T, H], the final-normed hidden states of the packed tokens; sequence s's
 * rows equal clef_backbone_prefill of its ids from `initial`.  No
 * counterpart in the reference (one request per call).
 */
size_t clef_backbone_varlen_workspace(const clef_backbone* b, int T, int nseq, int prefix_tokens);
int clef_backbone_prefill_varlen(clef_backbone* b, const int32_t* ids, const int32_t* cu_seqlens, int nseq,
                                 const void* initial, int initial_tokens, size_t initial_bytes, float* hidden,
                                 void* workspace, size_t workspace_bytes, void* stream);

/*
 * Cooperative cancellation and deadline, the reference's Control
 * (crates/core/src/models/mod.rs:45-59), checked where the reference checks
 * it: when a prefill starts (qwen.rs:344) and before each layer (qwen.rs:380).
 * `cancel` points to a host flag that another thread may set (nonzero =
 * cancel; NULL = never); `deadline` is an absolute time in seconds on the
 * clock of clef_monotonic_seconds() (0 = none).  A check that fails returns
 * CLEF_CANCELLED or CLEF_DEADLINE_EXCEEDED (Error::Cancelled /
 * Error::DeadlineExceeded) and launches nothing more; launches already
 * enqueued on the stream still run, and the outputs of a prefill that
 * returned an error are unspecified.  control NULL clears it.  The control
 * is read at every check, so the flag must outlive the prefills it governs.
 */
enum { CLEF_CANCELLED = -20, CLEF_DEADLINE_EXCEEDED = -21 };
typedef struct {
    const volatile int32_t* cancel;
    double deadline;
} clef_control;
int clef_backbone_set_control(clef_backbone* b, const clef_control* control);
double clef_monotonic_seconds(void);

/*
 * Diagnostics, the counterpart of the reference's test-only `measured!`
 * categories (crates/core/src/models/mod.rs:3-14, diagnostics.rs:43-96):
 * while enabled, prefills record a hipEvent pair on the stream around every
 * launch, by category.  clef_backbone_timings waits for those events, returns
 * per-category totals (milliseconds, launch counts, algorithmic flops and
 * algorithmic HBM bytes) and clears them.
 */
enum { CLEF_CAT_GEMM = 0, CLEF_CAT_SCAN, CLEF_CAT_ATTENTION, CLEF_CAT_CONV, CLEF_CAT_NORM,
       CLEF_CAT_OTHER, CLEF_CAT_COUNT };
int clef_backbone_enable_timing(clef_backbone* b, int enable);
int clef_backbone_timings(clef_backbone* b, double* ms, int* launches, double* flops,
                          double* bytes);

/* ---------------------------------------------------------------------- */
/* Weights on disk                                                         */
/* ---------------------------------------------------------------------- */
/*
 * Safetensors reader and device loader (the reference's Weights::load and
 * validate_header, models/weights.rs:26-104, 196-215).  clef_st_open maps a
 * file read-only and validates its header before returning: header length
 * at most 1 MiB, a JSON object of at most 2048 entries without duplicate
 * names, dtypes BF16 / F16 / F32, byte lengths equal to the shapes, and
 * tensors tiling the data section exactly; any violation is an error and no
 * handle is returned.  clef_st_info / clef_st_find describe the tensors
 * (name valid while the handle is open; shape8 receives up to 8 dims).
 * clef_st_load copies tensor i to the device and converts it there into
 * dtype_out (CLEF_F16 or CLEF_F32; BF16 -> F32 is exact, -> F16 rounds to
 * nearest even), using one tensor's worth of staging; it returns when the
 * data is in place.  The handle owns the mapping until clef_st_close.
 */
enum { CLEF_ST_BF16 = 2, CLEF_ST_F16 = 1, CLEF_ST_F32 = 0 };
typedef struct clef_safetensors clef_safetensors;
int clef_st_open(const char* path, clef_safetensors** out);
void clef_st_close(clef_safetensors* f);
int clef_st_count(const clef_safetensors* f);
int clef_st_info(const clef_safetensors* f, int i, const char** name, int* dtype, int* rank, int64_t* shape8);
int clef_st_find(const clef_safetensors* f, const char* name);
int clef_st_load(const clef_safetensors* f, int i, int dtype_out, void* dst, size_t dst_bytes, void* stream);

#ifdef __cplusplus
}
#endif
#endif

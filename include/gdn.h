/*
 * gdn.h -- C ABI of the MI355X (gfx950) Gated DeltaNet layer library, libgdn_hip.so.
 *
 * One Qwen3.5 Gated DeltaNet (GDN) linear-attention layer:
 *   x -> in_proj (q|k|v|z|a|b) -> causal conv1d (4 taps) + SiLU -> l2norm(q, k), g, beta
 *     -> gated delta rule (fp32 state per sequence and v-head) -> gated RMSNorm(o) * silu(z) -> out_proj
 *
 * Each entry point replaces one interface of the reference (paths relative to the reference root;
 * "9B/" = wormhole_n150/qwen3.5_9B/).  Conventions:
 *   - Every call returns GDN_OK (0) or a negative gdn_status; gdn_last_error() gives a message
 *     (thread-local).  Nothing aborts.
 *   - Tensors are device pointers, row-major, rows sequence-major (row m = b * T + t, 9B/gdn_layer.py:291).
 *     bf16 tensors are raw 16-bit words.  Weights use the HF [out_features, in_features] layout.
 *   - `stream` is a hipStream_t (NULL = the default stream).  Calls are asynchronous on that stream
 *     except gdn_layer_create/destroy, which synchronise the device.
 *   - A gdn_layer handle is not thread-safe.  Two sequences of one launch must not share a state slot.
 *   - Slot ids are device int32 arrays with values in [0, max_slots).  The library cannot read them on the
 *     host without a synchronisation, so the kernels check them: a sequence (or state-call entry) whose id
 *     is outside that range is skipped -- its states are not touched and its output rows are left
 *     unwritten.  Callers that hold the ids on the host check them first (the Python mirror raises
 *     GdnValueError before any launch).
 */
#ifndef GDN_H
#define GDN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct gdn_layer gdn_layer;
typedef struct gdn_stack gdn_stack;

typedef enum gdn_status {
    GDN_OK = 0,
    GDN_ERR_INVALID_ARG = -1,     /* null pointer, non-positive size */
    GDN_ERR_UNSUPPORTED = -2,     /* geometry the kernels do not implement */
    GDN_ERR_SHAPE = -3,           /* B, T, M or slot count outside the handle's limits */
    GDN_ERR_SLOT = -4,            /* slot id out of range */
    GDN_ERR_HIP = -5,             /* a HIP runtime call failed */
    GDN_ERR_OUT_OF_MEMORY = -6,   /* allocation at create time failed */
} gdn_status;

/* Layer geometry (HF Qwen3_5TextConfig fields; 9B/gdn_layer.py:58-64).  Supported: head_k_dim ==
 * head_v_dim in {32, 64, 128}, num_v_heads % num_k_heads == 0 with num_v_heads / num_k_heads <= 4,
 * conv_kernel == 4, hidden % 128 == 0, num_v_heads * head_v_dim % 128 == 0.  Other geometries are
 * GDN_ERR_UNSUPPORTED at create time. */
typedef struct gdn_dims {
    int hidden;        /* H: 4096 (9B), 1024 (0.8B) */
    int num_k_heads;   /* nk: 16 */
    int num_v_heads;   /* nv: 32 (9B), 16 (0.8B) */
    int head_k_dim;    /* dk: 128 */
    int head_v_dim;    /* dv: 128 */
    int conv_kernel;   /* 4 */
    float rms_norm_eps;/* 1e-6 */
} gdn_dims;

/* Weights of one layer in HF layouts (9B/README.md:44-52).  Pointers may be device or host memory;
 * gdn_layer_create copies them into the handle's own device layout. */
typedef struct gdn_weights {
    const void* in_proj_qkv;   /* bf16 [2*nk*dk + nv*dv, H] */
    const void* in_proj_z;     /* bf16 [nv*dv, H] */
    const void* in_proj_a;     /* bf16 [nv, H] */
    const void* in_proj_b;     /* bf16 [nv, H] */
    const float* conv1d;       /* fp32 [2*nk*dk + nv*dv, 4]  (conv1d.weight[:, 0, :]) */
    const float* A_log;        /* fp32 [nv] */
    const float* dt_bias;      /* fp32 [nv] */
    const float* norm_weight;  /* fp32 [dv] */
    const void* out_proj;      /* bf16 [H, nv*dv] */
} gdn_weights;

/* Weight storage of a layer: the reference's weight_dtype argument (9B/gdn_layer.py:55, 115-120: w_in and
 * w_out in ttnn.bfloat16, ttnn.bfloat8_b or ttnn.bfloat4_b, w_ab always bfloat16; 0.8B/gdn_l1.py:79-80). */
typedef enum gdn_weight_format {
    GDN_WEIGHTS_BF16 = 0,      /* the bf16 weights as given */
    GDN_WEIGHTS_FP8_E4M3 = 1,  /* in_proj q|k|v|z rows and out_proj as OCP E4M3 codes with one fp32 scale per
                                * output row (absmax / 448, see gdn_quantize_fp8); the a|b rows stay bf16.
                                * Activations and accumulation are unchanged (bf16 x bf16 MFMA, fp32). */
    GDN_WEIGHTS_MXFP4 = 2,     /* the counterpart of bfloat4_b: the same matrices as OCP MXFP4, E2M1 codes with
                                * one E8M0 scale per row and 32 columns (see gdn_quantize_mxfp4); the a|b
                                * rows stay bf16.
                                * Activations and accumulation are unchanged (bf16 x bf16 MFMA, fp32). */
    GDN_WEIGHTS_MXINT8 = 3,    /* the counterpart of bfloat8_b: the same matrices as OCP MXINT8, int8 codes
                                * worth code * 2^-6 with one E8M0 scale per row and 32 columns (see
                                * gdn_quantize_mxint8): 7 significant bits under a shared exponent, as
                                * bfloat8_b keeps; the a|b rows stay bf16.
                                * Activations and accumulation are unchanged (bf16 x bf16 MFMA, fp32). */
} gdn_weight_format;

/* ---- layer handle: mirrors Qwen35GatedDeltaNetTT (9B/gdn_layer.py:54-292) ------------------------ */

/* 9B/gdn_layer.py:55-78 (__init__), 90-127 (_prepare_weights), 137-151 (reset_state).
 * Copies the weights into the fused in_proj layout [q|k|v|z|a|b, H], allocates `max_slots` zeroed
 * state slots (recurrent [nv, dk, dv] fp32 + conv history) and a workspace for launches of up to
 * `max_tokens` rows (longer launches are split, 9B/gdn_layer.py:282-292). */
int gdn_layer_create(const gdn_dims* dims, const gdn_weights* weights, int max_slots, int max_tokens,
                     gdn_layer** out);

/* 9B/gdn_layer.py:55 with weight_dtype: gdn_layer_create with the weights stored in `weight_format`
 * (a gdn_weight_format), quantized on the device from the bf16 weights given. */
int gdn_layer_create_ex(const gdn_dims* dims, const gdn_weights* weights, int max_slots, int max_tokens,
                        int weight_format, gdn_layer** out);

/* The gdn_weight_format of a layer. */
int gdn_layer_weight_format(const gdn_layer* layer);

/* Element type of a layer's or a stack's output. */
typedef enum {
    GDN_OUT_BF16 = 0, /* bf16 (the default of a new handle) */
    GDN_OUT_FP32 = 1  /* fp32: the reference's layer output (9B/gdn_layer.py:272-276, ttnn.linear with
                       * dtype=ttnn.float32) and stack output (0.8B/gdn_l1.py:300, 336-339, fp32 rows) */
} gdn_out_dtype;

/* The element type (a gdn_out_dtype) of `out` in gdn_layer_forward, gdn_layer_forward_varlen and
 * gdn_out_proj of this layer, for calls issued after it.  Both types store the same fp32 sums of the
 * out_proj; the bf16 output is the fp32 one rounded to nearest even.  The state, the workspace and the
 * activations inside the layer are the same for both.  A split launch (B > 1 and T > max_tokens / B) with
 * fp32 output needs gdn_layer_proj_width() >= hidden (true of every Qwen3.5 shape), else it fails with
 * GDN_ERR_UNSUPPORTED. */
int gdn_layer_set_output_dtype(gdn_layer* layer, int out_dtype);

/* The gdn_out_dtype of a layer's output. */
int gdn_layer_output_dtype(const gdn_layer* layer);

int gdn_layer_destroy(gdn_layer* layer);

/* 9B/gdn_layer.py:282-292 (__call__) and 244-280 (_forward_rows).
 * x: bf16 [B*T, H]; out: [B*T, H] of the layer's output type (bf16 unless gdn_layer_set_output_dtype).
 * slot_ids: device int32 [B] (state slot of sequence b), or NULL for slots 0..B-1.  Continues every
 * sequence from its slot's conv and recurrent state. */
int gdn_layer_forward(gdn_layer* layer, const void* x, int B, int T, const int* slot_ids, void* out,
                      void* stream);

/* Variable-length launch (no counterpart in the reference, which fixes one batch geometry per handle and
 * maps row -> slot as m / T, 9B/kernels/layer_compute.cpp:231): n_seqs sequences of different lengths in
 * one call, e.g. prefills and decode streams of a continuous batch.  x: bf16 [cu_seqlens[n_seqs], H], out: the
 * same rows of the layer's output type; sequence i is rows [cu_seqlens[i], cu_seqlens[i+1]) (host int32 [n_seqs + 1], cu_seqlens[0] = 0, at most
 * max_tokens rows) and continues slot slot_ids[i] (device int32 [n_seqs], or NULL for slots 0..n_seqs-1).
 * The in_proj and out_proj run once over all rows; runs of consecutive equal-length sequences share one
 * launch of the middle of the layer.  The result of each sequence equals its own gdn_layer_forward up to
 * the rounding of the projection kernel chosen for the total row count. */
int gdn_layer_forward_varlen(gdn_layer* layer, const void* x, int n_seqs, const int* cu_seqlens,
                             const int* slot_ids, void* out, void* stream);

/* 9B/gdn_layer.py:137-151 (reset_state): zero the states of `n` slots (device ids, NULL = the first n). */
int gdn_state_reset(gdn_layer* layer, const int* slot_ids, int n, void* stream);

/* 9B/gdn_layer.py:153-157 (get_recurrent_state): copy the states of n slots out.
 * rec: fp32 [n, nv, dk, dv]; conv: fp32 [n, conv_dim, 3], time order (entry 2 = newest); either may be NULL. */
int gdn_state_get(gdn_layer* layer, const int* slot_ids, int n, float* rec, float* conv, void* stream);

/* 9B/gated_delta_l1.py:156-173 (reset_state(initial_state)): seed the states of n slots.  rec and conv as
 * in gdn_state_get; a NULL rec leaves the recurrent state, a NULL conv zeroes the conv history. */
int gdn_state_set(gdn_layer* layer, const int* slot_ids, int n, const float* rec, const float* conv, void* stream);

/* Device addresses of the resident state buffers (for address-stability checks,
 * 9B/test_gated_delta_l1.py:81-92); any output may be NULL.  rec: [max_slots, nv, dk, dv] fp32.
 * conv: the conv history rings, [max_slots, nk, 4, 2 dk + R dv] fp32 with R = nv / nk: per slot and k-head
 * group kh the pre-conv inputs of the group's channels (q and k of kh, then v of the v-heads R kh ..
 * R kh + R - 1), the input of token time tau at entry tau % 4.  conv_pos: int32 [max_slots, nv], pos = tokens
 * seen % 4 per v-head (equal for all v-heads of a slot); the window of the next token, time order j = 0
 * (oldest) .. 2, is entry (pos + 1 + j) % 4.  A launch of T tokens writes only its last min(T, 3) inputs, one
 * entry per token, and advances pos by T. */
int gdn_layer_state_buffers(gdn_layer* layer, void** rec, void** conv, void** conv_pos);

/* Stage timing with HIP events recorded on the launch stream at the stage boundaries of every launch of
 * the layer (no counterpart in the reference, whose benches read the tt-metal device profiler,
 * wormhole_n150/qwen3.5_0.8B/bench_decode.py:35-37).  A launch is one gdn_layer_forward or
 * gdn_layer_forward_varlen call of at most max_tokens rows; a longer gdn_layer_forward call is split into
 * launches of at most max_tokens rows and records one set per launch.  gdn_layer_profile(layer, n) starts
 * recording for up to n launches (n = 0 stops); gdn_layer_profile_read synchronises on the last event and
 * writes the summed milliseconds per stage: ms[0] in_proj, ms[1] mixer (conv .. gated RMSNorm),
 * ms[2] out_proj, ms[3] whole launch; *calls = number of launches recorded. */
int gdn_layer_profile(gdn_layer* layer, int max_calls);
int gdn_layer_profile_read(gdn_layer* layer, double* ms, int* calls);

/* Width of the fused projection row, conv_dim + nv*dv + 2*nv (q | k | v | z | a | b). */
int gdn_layer_proj_width(const gdn_layer* layer);

/* ---- per-op entries: the five stages of the layer, on caller-owned device buffers --------------- */

/* in_proj: 9B/gdn_layer.py:255-258 (q|k|v|z) + 259 (a|b) as one projection.
 * x bf16 [M, H] -> P fp32 [M, gdn_layer_proj_width()] = x [W_qkv; W_z; W_a; W_b]^T. */
int gdn_in_proj(gdn_layer* layer, const void* x, int M, float* P, void* stream);

/* Front end: 9B/kernels/layer_compute.cpp C1-C4 (74-222) with layer_reader.cpp:103-124,184-197.
 * Causal conv1d + SiLU of the q|k|v part of P (continuing each slot's conv history, which it advances),
 * l2norm, g = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b).
 * qn, kn: fp32 [M, nk, dk] (qn scaled by dk^-0.5); v: fp32 [M, nv, dv]; g, beta: fp32 [M, nv]. */
int gdn_conv_front(gdn_layer* layer, const float* P, int B, int T, const int* slot_ids, float* qn, float* kn,
                   float* v, float* g, float* beta, void* stream);

/* Recurrence: 9B/kernels/layer_compute.cpp C5 (224-285); 9B/reference.py:28-34.
 * On normalised inputs from gdn_conv_front, continuing each slot's recurrent state.  o: fp32 [M, nv, dv].
 * Launches of more than 64 tokens per sequence use the chunk-64 form (HF torch_chunk_gated_delta_rule,
 * modeling_qwen3_5.py:248-328) when dk == dv == 128, otherwise the token loop. */
int gdn_delta_rule(gdn_layer* layer, const float* qn, const float* kn, const float* v, const float* g,
                   const float* beta, int B, int T, const int* slot_ids, float* o, void* stream);

/* Gated RMSNorm: 9B/kernels/layer_compute.cpp C6 (287-395); HF Qwen3_5RMSNormGated.
 * o fp32 [M, nv*dv], z fp32 rows of stride z_stride (the z block of P) -> y bf16 [M, nv*dv]. */
int gdn_gated_rmsnorm(gdn_layer* layer, const float* o, const float* z, int z_stride, int M, void* y,
                      void* stream);

/* out_proj: 9B/gdn_layer.py:272-276.  y bf16 [M, nv*dv] -> out [M, H] of the layer's output type
 * (gdn_layer_set_output_dtype). */
int gdn_out_proj(gdn_layer* layer, const void* y, int M, void* out, void* stream);

/* ---- layer stack: mirrors Qwen35_08B_GDNStackL1 (wormhole_n150/qwen3.5_0.8B/gdn_l1.py:207-341) ---- */

/* n_layers layers of one geometry (weights[i] = layer i, as in gdn_layer_create), run back to back: the
 * output of layer i is the input of layer i + 1, each layer with its own `max_slots` state slots
 * (gdn_l1.py:330-341: GDN mixers only).  inter_norm != 0 adds the decoder RMSNorm between layers,
 * y = x rsqrt(mean(x^2) + eps) (1 + w) (HF Qwen3_5RMSNorm, modeling_qwen3_5.py:720-734), with w =
 * norm_weights[i] (fp32 [H], host or device) after layer i, or w = 0 where norm_weights or the entry is
 * NULL; no norm follows the last layer.  The layers share one workspace for `max_tokens` rows. */
int gdn_stack_create(const gdn_dims* dims, const gdn_weights* weights, int n_layers, int inter_norm,
                     const float* const* norm_weights, int max_slots, int max_tokens, gdn_stack** out);
/* The same with every layer's weights in `weight_format` (gdn_l1.py:79-80, the stack's weight dtype). */
int gdn_stack_create_ex(const gdn_dims* dims, const gdn_weights* weights, int n_layers, int inter_norm,
                        const float* const* norm_weights, int max_slots, int max_tokens, int weight_format,
                        gdn_stack** out);
int gdn_stack_destroy(gdn_stack* stack);

/* The handle of layer i, for the state calls (gdn_state_*) and per-op entries.  Owned by the stack. */
int gdn_stack_layer(gdn_stack* stack, int i, gdn_layer** layer);

/* The element type (a gdn_out_dtype, bf16 for a new stack) of the output of gdn_stack_forward(_varlen)
 * calls that run the stack's last layer; gdn_l1.py:300, 336-339 returns fp32 rows (GDN_OUT_FP32).  The
 * activations between layers stay bf16, and so does the output of a call that ends before the last layer
 * (the input of the next call).  A layer's own setting (gdn_layer_set_output_dtype) does not apply inside
 * the stack. */
int gdn_stack_set_output_dtype(gdn_stack* stack, int out_dtype);

/* gdn_l1.py:294-341 (forward_device / __call__(hidden_states, layers)): layers [first, first + count) on
 * x bf16 [B*T, H] -> out [B*T, H], of the stack's output type (gdn_stack_set_output_dtype) when the call
 * runs the stack's last layer and bf16 otherwise; slot_ids as in gdn_layer_forward.  Launches of more than
 * max_tokens rows run token blocks of at most max_tokens rows through all the layers in turn
 * (B <= max_tokens). */
int gdn_stack_forward(gdn_stack* stack, const void* x, int B, int T, const int* slot_ids, int first, int count,
                      void* out, void* stream);

/* The same over a variable-length launch (see gdn_layer_forward_varlen; at most max_tokens rows). */
int gdn_stack_forward_varlen(gdn_stack* stack, const void* x, int n_seqs, const int* cu_seqlens,
                             const int* slot_ids, int first, int count, void* out, void* stream);

/* ---- standalone ops ------------------------------------------------------------------------------ */

/* Recurrence-only op: mirrors GatedDeltaRuleL1.__call__ (9B/gated_delta_l1.py:260-272, packing 90-122)
 * and the CPU oracle recurrent_gated_delta_rule (9B/reference.py:11-35).
 * q, k: fp32 [B, T, Hk, dk]; v: fp32 [B, T, Hv, dv]; g (log decay), beta: fp32 [B, T, Hv];
 * state: fp32 [B, Hv, dk, dv], read as the initial state and overwritten with the final state;
 * o: fp32 [B, T, Hv, dv].  use_qk_l2norm: l2-normalise q and k (eps 1e-6); scale <= 0 means dk^-0.5. */
int gdn_delta_rule_fla(const float* q, const float* k, const float* v, const float* g, const float* beta, int B,
                       int T, int Hk, int Hv, int dk, int dv, float* state, int use_qk_l2norm, float scale,
                       float* o, void* stream);

/* Bytes of device workspace that gdn_delta_rule_fla_ws needs to run this launch in the chunk-64 form (the
 * counterpart of HF's torch_chunk_gated_delta_rule, HF:248-328, which the reference's prefill of a whole
 * prompt evaluates); 0 when the launch runs the token loop anyway (T <= 64, head dims other than 128 x 128,
 * or a bad shape). */
size_t gdn_delta_rule_fla_workspace_size(int B, int T, int Hv, int dk, int dv);

/* gdn_delta_rule_fla with a caller-owned device workspace (nothing is allocated).  When
 * gdn_delta_rule_fla_workspace_size(B, T, Hv, dk, dv) > 0 and workspace_bytes is at least that, the launch
 * runs the chunk-64 form: a parallel pass per (sequence, v-head, 64-token chunk), then one sequential pass
 * over the chunks.  Same arguments, layouts and results (within fp32 rounding) as gdn_delta_rule_fla.
 * workspace NULL: the token loop, exactly gdn_delta_rule_fla.  A non-NULL workspace smaller than the size
 * above is GDN_ERR_SHAPE.  Calls that share one workspace must not overlap. */
int gdn_delta_rule_fla_ws(const float* q, const float* k, const float* v, const float* g, const float* beta,
                          int B, int T, int Hk, int Hv, int dk, int dv, float* state, int use_qk_l2norm,
                          float scale, float* o, void* workspace, size_t workspace_bytes, void* stream);

/* No counterpart in the reference: gdn_delta_rule_fla_ws for callers that cannot allocate device memory
 * (code under HIP-graph capture, serving loops and harnesses that forbid hipMalloc).  The chunk-64 workspace
 * is a static device array of GDN_NOALLOC_SCRATCH_BYTES that the library holds on every device it runs on
 * until the process ends; nothing is allocated and no workspace is passed.  Launches that need more
 * (B * Hv * ceil(T / 64) above 408 for 128-wide heads) return GDN_ERR_SHAPE; launches the token loop runs
 * (T <= 64, other head sizes) need none.  Same arguments, layouts and results as gdn_delta_rule_fla_ws with a
 * large enough workspace.  All calls on one device share that device's array: calls that overlap in time on
 * one device (other streams, other threads) race; the array keeps the last call's contents and needs no
 * clearing (every call writes all it reads). */
#define GDN_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int gdn_delta_rule_fla_noalloc(const float* q, const float* k, const float* v, const float* g, const float* beta,
                               int B, int T, int Hk, int Hv, int dk, int dv, float* state, int use_qk_l2norm,
                               float scale, float* o, void* stream);

/* Projection y[M, N] = x[M, K] . w[N, K]^T, bf16 inputs, fp32 accumulation (the ttnn.linear call sites
 * 9B/gdn_layer.py:255, 259, 272).  out_fp32 != 0: y is fp32, else bf16.  K % 128 == 0. */
int gdn_linear_bf16(const void* x, const void* w, int M, int N, int K, void* y, int out_fp32, void* stream);

/* The E4M3 weight quantizer of GDN_WEIGHTS_FP8_E4M3 (the reference's host-side conversion to bfloat8_b,
 * ttnn.from_torch(..., dtype=weight_dtype) at 9B/gdn_layer.py:115-120, re-specified for OCP E4M3):
 * w bf16 [N, K] (device) -> q uint8 [N, K] E4M3 codes, scale fp32 [N], with scale[n] = max_k |w[n, k]| / 448
 * (1 for an all-zero row) and q[n, k] = round-to-nearest-even(w[n, k] / scale[n]), saturating at +-448.
 * Row n of the dequantized matrix is decode(q[n, :]) * scale[n]. */
int gdn_quantize_fp8(const void* w, int N, int K, void* q, float* scale, void* stream);

/* The MXFP4 weight quantizer of GDN_WEIGHTS_MXFP4 (the reference's conversion to bfloat4_b, ttnn.from_torch(...,
 * dtype=weight_dtype) at 0.8B/gdn_l1.py:79-80, re-specified for OCP MXFP4): w bf16 [N, K] (device, K % 32 ==
 * 0) -> q uint8 [N, K / 2] E2M1 codes, two per byte (column 2i in the low nibble), and scale uint8 [N, K / 32]
 * E8M0 codes, block j of row n (columns 32 j .. 32 j + 31) scaled by X = 2^(floor(log2 max |w|) - 2)
 * (exponent clamped to [-127, 127], code = exponent + 127; 0 for an all-zero block) and each value coded as
 * round-to-nearest-even(w / X) on the E2M1 grid {0, 0.5, 1, 1.5, 2, 3, 4, 6}, saturating at +-6.  The
 * dequantized value is decode(code) * 2^(scale code - 127). */
int gdn_quantize_mxfp4(const void* w, int N, int K, void* q, void* scale, void* stream);

/* The MXINT8 weight quantizer of GDN_WEIGHTS_MXINT8 (the reference's conversion to bfloat8_b, ttnn.from_torch(...,
 * dtype=weight_dtype) at 9B/gdn_layer.py:115-120 and 0.8B/gdn_l1.py:79-80, re-specified for OCP MXINT8): w bf16
 * [N, K] (device, K % 32 == 0) -> q int8 [N, K] codes and scale uint8 [N, K / 32] E8M0 codes, block j of row n
 * (columns 32 j .. 32 j + 31) scaled by X = 2^floor(log2 max |w|) (exponent clamped to [-127, 127], code =
 * exponent + 127; 0 for an all-zero block) and each value coded as round-to-nearest-even(64 w / X) saturated
 * to [-128, 127].  The dequantized value is code * 2^(scale code - 133). */
int gdn_quantize_mxint8(const void* w, int N, int K, void* q, void* scale, void* stream);

/* Message of the last failed call on this thread ("" if none). */
const char* gdn_last_error(void);

/* Library version, major * 10000 + minor * 100 + patch. */
int gdn_version(void);

#ifdef __cplusplus
}
#endif

#endif /* GDN_H */

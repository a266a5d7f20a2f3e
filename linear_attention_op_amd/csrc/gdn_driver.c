/*
 * gdn_driver -- a C host driver of the layer ABI (include/gdn.h): no Python, no torch.
 *
 * Builds one Gated DeltaNet layer of the 9B or 0.8B geometry from seeded synthetic weights held in host
 * memory (HF layouts, as gdn_layer_create takes them), prefills one sequence, then runs batched single-token
 * decode steps on a HIP stream and times them with HIP events after the clocks have settled.  It checks what
 * a caller without a reference can check: every output and state value is finite, the state buffers keep
 * their addresses, the fp32 and bf16 outputs of one step agree to bf16 rounding, and the error paths return
 * their codes with a message.  Prints one line of key = value pairs; exit status 0 when every check passed,
 * 1 when one failed, 2 when no GPU is present or an argument is wrong.
 *
 *     gdn_driver [--shape 9b|0.8b] [--batch B] [--steps N] [--prefill T] [--weights bf16|fp8|mxfp4|mxint8]
 *
 * The mirror of this flow in the reference is its decode benchmark (wormhole_n150/qwen3.5_0.8B/
 * bench_decode.py:24-60: build the layer, warm up, time traced decode steps).
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "../../include/gdn.h"

static int failures = 0;

static void check(int ok, const char* what) {
    if (!ok) {
        fprintf(stderr, "gdn_driver: check failed: %s (%s)\n", what, gdn_last_error());
        ++failures;
    }
}

#define HIPCHK(x)                                                                              \
    do {                                                                                       \
        hipError_t e_ = (x);                                                                   \
        if (e_ != hipSuccess) {                                                                \
            fprintf(stderr, "gdn_driver: %s failed: %s\n", #x, hipGetErrorString(e_));         \
            exit(1);                                                                           \
        }                                                                                      \
    } while (0)

/* deterministic uniform [0, 1) */
static uint64_t rng = 0x9e3779b97f4a7c15ull;
static double urand(void) {
    rng = rng * 6364136223846793005ull + 1442695040888963407ull;
    return (double)(rng >> 11) * (1.0 / 9007199254740992.0);
}
/* standard normal (Box-Muller) */
static double nrand(void) {
    const double u = urand() + 1e-300, v = urand();
    return sqrt(-2.0 * log(u)) * cos(6.283185307179586 * v);
}
/* float -> bf16 bits, round to nearest even */
static uint16_t bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
static uint16_t* bf16_normal(size_t n, double std) {
    uint16_t* p = (uint16_t*)malloc(n * sizeof(uint16_t));
    for (size_t i = 0; i < n; ++i) p[i] = bf16((float)(nrand() * std));
    return p;
}
static int all_finite_f32(const float* p, size_t n) {
    for (size_t i = 0; i < n; ++i)
        if (!isfinite(p[i])) return 0;
    return 1;
}

int main(int argc, char** argv) {
    const char* shape = "9b";
    int B = 64, steps = 200, T = 1024, fmt = GDN_WEIGHTS_BF16;
    for (int i = 1; i < argc; ++i) {
        if (!strcmp(argv[i], "--shape") && i + 1 < argc) shape = argv[++i];
        else if (!strcmp(argv[i], "--batch") && i + 1 < argc) B = atoi(argv[++i]);
        else if (!strcmp(argv[i], "--steps") && i + 1 < argc) steps = atoi(argv[++i]);
        else if (!strcmp(argv[i], "--prefill") && i + 1 < argc) T = atoi(argv[++i]);
        else if (!strcmp(argv[i], "--weights") && i + 1 < argc) {
            const char* w = argv[++i];
            fmt = !strcmp(w, "fp8") ? GDN_WEIGHTS_FP8_E4M3 : !strcmp(w, "mxfp4") ? GDN_WEIGHTS_MXFP4
                  : !strcmp(w, "mxint8") ? GDN_WEIGHTS_MXINT8 : !strcmp(w, "bf16") ? GDN_WEIGHTS_BF16 : -1;
        } else {
            fprintf(stderr, "usage: gdn_driver [--shape 9b|0.8b] [--batch B] [--steps N] [--prefill T] "
                            "[--weights bf16|fp8|mxfp4|mxint8]\n");
            return 2;
        }
    }
    gdn_dims d;
    if (!strcmp(shape, "9b")) d = (gdn_dims){4096, 16, 32, 128, 128, 4, 1e-6f};
    else if (!strcmp(shape, "0.8b")) d = (gdn_dims){1024, 16, 16, 128, 128, 4, 1e-6f};
    else {
        fprintf(stderr, "gdn_driver: shape %s (9b or 0.8b)\n", shape);
        return 2;
    }
    if (B <= 0 || steps <= 0 || T < 0 || fmt < 0) {
        fprintf(stderr, "gdn_driver: bad batch, steps, prefill length or weight format\n");
        return 2;
    }
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev == 0) {
        fprintf(stderr, "gdn_driver: no HIP device\n");
        return 2;
    }
    HIPCHK(hipSetDevice(0));

    const int H = d.hidden, nv = d.num_v_heads, dk = d.head_k_dim, dv = d.head_v_dim;
    const int Kd = d.num_k_heads * dk, Vd = nv * dv, C = 2 * Kd + Vd;

    /* host weights, HF layouts: projections N(0, 0.02) in bf16; taps N(0, 0.02); A_log = log U(0, 16),
     * dt_bias U(-1, 1), norm weight U(0.5, 1.5) */
    uint16_t* w_qkv = bf16_normal((size_t)C * H, 0.02);
    uint16_t* w_z = bf16_normal((size_t)Vd * H, 0.02);
    uint16_t* w_a = bf16_normal((size_t)nv * H, 0.02);
    uint16_t* w_b = bf16_normal((size_t)nv * H, 0.02);
    uint16_t* w_out = bf16_normal((size_t)H * Vd, 0.02);
    float* conv = (float*)malloc((size_t)C * 4 * sizeof(float));
    for (size_t i = 0; i < (size_t)C * 4; ++i) conv[i] = (float)(nrand() * 0.02);
    float* A_log = (float*)malloc(nv * sizeof(float));
    float* dt_bias = (float*)malloc(nv * sizeof(float));
    float* norm_w = (float*)malloc(dv * sizeof(float));
    for (int i = 0; i < nv; ++i) A_log[i] = (float)log(fmax(urand() * 16.0, 1e-9)), dt_bias[i] = (float)(2 * urand() - 1);
    for (int i = 0; i < dv; ++i) norm_w[i] = (float)(urand() + 0.5);
    const gdn_weights w = {w_qkv, w_z, w_a, w_b, conv, A_log, dt_bias, norm_w, w_out};

    const int max_tokens = T > B ? T : B;
    gdn_layer* L = NULL;
    int rc = gdn_layer_create_ex(&d, &w, B, max_tokens, fmt, &L);
    if (rc) {
        fprintf(stderr, "gdn_driver: gdn_layer_create_ex: %d (%s)\n", rc, gdn_last_error());
        return 1;
    }
    check(gdn_layer_weight_format(L) == fmt, "weight format");

    hipStream_t st;
    HIPCHK(hipStreamCreate(&st));
    void *x, *out, *out16;
    float* rec;
    int* slot0;
    const size_t rows = (size_t)max_tokens;
    HIPCHK(hipMalloc(&x, rows * H * sizeof(uint16_t)));
    HIPCHK(hipMalloc(&out, rows * H * sizeof(float)));
    HIPCHK(hipMalloc(&out16, (size_t)B * H * sizeof(uint16_t)));
    HIPCHK(hipMalloc((void**)&rec, (size_t)nv * dk * dv * sizeof(float)));
    HIPCHK(hipMalloc((void**)&slot0, sizeof(int)));
    HIPCHK(hipMemset(slot0, 0, sizeof(int)));
    {
        uint16_t* hx = bf16_normal(rows * H, 1.0);
        HIPCHK(hipMemcpy(x, hx, rows * H * sizeof(uint16_t), hipMemcpyHostToDevice));
        free(hx);
    }
    void *rec_addr0 = NULL, *conv_addr0 = NULL;
    check(gdn_layer_state_buffers(L, &rec_addr0, &conv_addr0, NULL) == GDN_OK && rec_addr0 && conv_addr0,
          "state buffers");

    /* prefill: one sequence of T tokens into slot 0, bf16 output */
    hipEvent_t e0, e1;
    HIPCHK(hipEventCreate(&e0));
    HIPCHK(hipEventCreate(&e1));
    float prefill_ms = 0.f;
    if (T > 0) {
        HIPCHK(hipEventRecord(e0, st));
        check(gdn_layer_forward(L, x, 1, T, slot0, out, st) == GDN_OK, "prefill");
        HIPCHK(hipEventRecord(e1, st));
        HIPCHK(hipEventSynchronize(e1));
        HIPCHK(hipEventElapsedTime(&prefill_ms, e0, e1));
    }

    /* one decode step with fp32 output and the same step (same states) with bf16 output */
    check(gdn_layer_set_output_dtype(L, GDN_OUT_FP32) == GDN_OK && gdn_layer_output_dtype(L) == GDN_OUT_FP32,
          "fp32 output");
    float *drec, *dconv;
    HIPCHK(hipMalloc((void**)&drec, (size_t)B * nv * dk * dv * sizeof(float)));
    HIPCHK(hipMalloc((void**)&dconv, (size_t)B * C * 3 * sizeof(float)));
    check(gdn_state_get(L, NULL, B, drec, dconv, st) == GDN_OK, "state get");
    check(gdn_layer_forward(L, x, B, 1, NULL, out, st) == GDN_OK, "decode step (fp32 out)");
    check(gdn_state_set(L, NULL, B, drec, dconv, st) == GDN_OK, "state set");
    check(gdn_layer_set_output_dtype(L, GDN_OUT_BF16) == GDN_OK, "bf16 output");
    check(gdn_layer_forward(L, x, B, 1, NULL, out16, st) == GDN_OK, "decode step (bf16 out)");
    HIPCHK(hipStreamSynchronize(st));
    {
        float* o32 = (float*)malloc((size_t)B * H * sizeof(float));
        uint16_t* o16 = (uint16_t*)malloc((size_t)B * H * sizeof(uint16_t));
        HIPCHK(hipMemcpy(o32, out, (size_t)B * H * sizeof(float), hipMemcpyDeviceToHost));
        HIPCHK(hipMemcpy(o16, out16, (size_t)B * H * sizeof(uint16_t), hipMemcpyDeviceToHost));
        size_t same = 0;
        for (size_t i = 0; i < (size_t)B * H; ++i) same += bf16(o32[i]) == o16[i];
        check(all_finite_f32(o32, (size_t)B * H), "decode output finite");
        check(same == (size_t)B * H, "bf16 output = fp32 output rounded to nearest even");
        free(o32);
        free(o16);
    }

    /* timed decode: settle the clocks (0.3 s of steps), then `steps` steps */
    int settle = 0;
    {
        float ms = 0.f;
        HIPCHK(hipEventRecord(e0, st));
        while (ms < 300.f) {
            for (int i = 0; i < 50; ++i) gdn_layer_forward(L, x, B, 1, NULL, out16, st);
            settle += 50;
            HIPCHK(hipEventRecord(e1, st));
            HIPCHK(hipEventSynchronize(e1));
            HIPCHK(hipEventElapsedTime(&ms, e0, e1));
        }
    }
    HIPCHK(hipEventRecord(e0, st));
    for (int i = 0; i < steps; ++i) rc |= gdn_layer_forward(L, x, B, 1, NULL, out16, st);
    HIPCHK(hipEventRecord(e1, st));
    HIPCHK(hipEventSynchronize(e1));
    check(rc == GDN_OK, "timed decode steps");
    float decode_ms = 0.f;
    HIPCHK(hipEventElapsedTime(&decode_ms, e0, e1));
    const double us = decode_ms * 1e3 / steps;

    /* the state of slot 0 after every step: finite, at the same address */
    check(gdn_state_get(L, slot0, 1, rec, NULL, st) == GDN_OK, "state get (slot 0)");
    HIPCHK(hipStreamSynchronize(st));
    {
        float* hrec = (float*)malloc((size_t)nv * dk * dv * sizeof(float));
        HIPCHK(hipMemcpy(hrec, rec, (size_t)nv * dk * dv * sizeof(float), hipMemcpyDeviceToHost));
        check(all_finite_f32(hrec, (size_t)nv * dk * dv), "state finite");
        free(hrec);
    }
    void *rec_addr1 = NULL, *conv_addr1 = NULL;
    gdn_layer_state_buffers(L, &rec_addr1, &conv_addr1, NULL);
    check(rec_addr1 == rec_addr0 && conv_addr1 == conv_addr0, "state buffers stay in place");

    /* error paths: codes and a message, nothing launched */
    check(gdn_layer_forward(NULL, x, 1, 1, NULL, out, st) == GDN_ERR_INVALID_ARG && gdn_last_error()[0],
          "NULL layer is GDN_ERR_INVALID_ARG");
    check(gdn_layer_forward(L, x, 0, 1, NULL, out, st) == GDN_ERR_SHAPE, "B = 0 is GDN_ERR_SHAPE");
    check(gdn_layer_forward(L, x, B + 1, 1, NULL, out, st) != GDN_OK, "more sequences than slots is an error");
    check(gdn_layer_set_output_dtype(L, 7) == GDN_ERR_INVALID_ARG, "unknown output type");

    printf("shape=%s batch=%d weights=%d prefill_tokens=%d prefill_ms=%.3f decode_steps=%d settle_steps=%d "
           "decode_us_per_step=%.2f decode_tok_per_s=%.0f checks_failed=%d\n",
           shape, B, fmt, T, prefill_ms, steps, settle, us, B / (us * 1e-6), failures);

    gdn_layer_destroy(L);
    hipFree(x), hipFree(out), hipFree(out16), hipFree(rec), hipFree(slot0), hipFree(drec), hipFree(dconv);
    hipEventDestroy(e0), hipEventDestroy(e1), hipStreamDestroy(st);
    free(w_qkv), free(w_z), free(w_a), free(w_b), free(w_out), free(conv), free(A_log), free(dt_bias), free(norm_w);
    return failures ? 1 : 0;
}

// C ABI of the Gated DeltaNet library (include/gdn.h): layer handle, dispatch, state slots.
//
// The handle mirrors Qwen35GatedDeltaNetTT (wormhole_n150/qwen3.5_9B/gdn_layer.py:54-292): it owns the
// weights (re-laid out once at create), per-slot resident states and the launch workspace, and a
// forward call is  in_proj -> mixer -> out_proj.  Launches longer than the workspace are split by
// tokens with the states carried across, like the reference's 128-row launches (gdn_layer.py:282-292).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/gdn.h"
#include "gdn_common.h"

using gdn::u16;

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

#define HIP_OK(expr)                                                                              \
    do {                                                                                          \
        hipError_t e_ = (expr);                                                                   \
        if (e_ != hipSuccess) return fail(GDN_ERR_HIP, "%s: %s", #expr, hipGetErrorString(e_));   \
    } while (0)

// Prefills longer than this many tokens per sequence use the token-parallel front end + chunked rule.
constexpr int kFusedMaxT = 64;

bool supported_head_dim(int d) { return d == 32 || d == 64 || d == 128; }

}  // namespace

struct gdn_layer {
    gdn_dims d{};
    int Kd = 0, Vd = 0, CD = 0, NP = 0, CH = 0;
    int max_slots = 0, max_tokens = 0;
    std::vector<void*> allocs;

    u16* w_in = nullptr;      // [NP, H]  rows q | k | v | z | a | b, W_FRAG layout
    u16* w_out = nullptr;     // [H, Vd] W_FRAG layout
    float4* conv_w = nullptr; // [CD] taps
    float* neg_A = nullptr;   // [nv]
    float* dt_bias = nullptr; // [nv]
    float* norm_w = nullptr;  // [dv]
    float* rec = nullptr;     // [slots, nv, dk, dv]
    float* conv = nullptr;    // [slots, nv, 3, CH] conv history, time order

    // workspace, sized for max_tokens rows
    u16* x_ws = nullptr;      // [max_tokens, H] gathered input rows when a launch is split
    u16* x_frag = nullptr;    // [64, H] decode input in W_FRAG layout
    u16* out_ws = nullptr;    // [max_tokens, H]
    float* P = nullptr;       // [max_tokens, NP]
    float* qn = nullptr;      // [max_tokens, Kd]
    float* kn = nullptr;      // [max_tokens, Kd]
    float* v = nullptr;       // [max_tokens, Vd]
    float* g = nullptr;       // [max_tokens, nv]
    float* beta = nullptr;    // [max_tokens, nv]
    float* o = nullptr;       // [max_tokens, Vd]
    u16* y = nullptr;         // [max_tokens, Vd]
    void* chunk_ws = nullptr;
    size_t chunk_ws_bytes = 0;

    // stage timing: 4 events per recorded call (start, after in_proj, after mixer, after out_proj)
    std::vector<hipEvent_t> prof_events;
    int prof_max = 0, prof_calls = 0;

    template <typename Tp>
    hipError_t alloc(Tp** p, size_t count) {
        void* q = nullptr;
        hipError_t e = hipMalloc(&q, count * sizeof(Tp) > 0 ? count * sizeof(Tp) : 16);
        if (e == hipSuccess) allocs.push_back(q);
        *p = static_cast<Tp*>(q);
        return e;
    }
    void prof_free() {
        for (hipEvent_t e : prof_events) (void)hipEventDestroy(e);
        prof_events.clear();
        prof_max = prof_calls = 0;
    }
    hipEvent_t prof_event(int stage) const {
        return prof_calls < prof_max ? prof_events[(size_t)prof_calls * 4 + stage] : nullptr;
    }
    ~gdn_layer() {
        prof_free();
        for (void* p : allocs) (void)hipFree(p);
    }
};

namespace {

int check_dims(const gdn_dims* d) {
    if (!d) return fail(GDN_ERR_INVALID_ARG, "dims is NULL");
    if (d->hidden <= 0 || d->num_k_heads <= 0 || d->num_v_heads <= 0)
        return fail(GDN_ERR_INVALID_ARG, "non-positive geometry");
    if (d->head_k_dim != d->head_v_dim || !supported_head_dim(d->head_k_dim))
        return fail(GDN_ERR_UNSUPPORTED, "head dims %d x %d: need dk == dv in {32, 64, 128}", d->head_k_dim,
                    d->head_v_dim);
    if (d->num_v_heads % d->num_k_heads)
        return fail(GDN_ERR_UNSUPPORTED, "num_v_heads %d is not a multiple of num_k_heads %d", d->num_v_heads,
                    d->num_k_heads);
    if (d->conv_kernel != 4) return fail(GDN_ERR_UNSUPPORTED, "conv_kernel %d (only 4)", d->conv_kernel);
    if (d->hidden % 128) return fail(GDN_ERR_UNSUPPORTED, "hidden %d is not a multiple of 128", d->hidden);
    if ((d->num_v_heads * d->head_v_dim) % 128)
        return fail(GDN_ERR_UNSUPPORTED, "value dim %d is not a multiple of 128", d->num_v_heads * d->head_v_dim);
    return GDN_OK;
}

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

// Recurrence dispatch: launches of more than kFusedMaxT tokens per sequence take the chunk-64 form
// (when the head size has it and the workspace holds the launch), shorter ones the token loop.
hipError_t run_delta(gdn_layer* L, const gdn::DeltaArgs& r, hipStream_t st) {
    const gdn_dims& d = L->d;
    if (r.T > kFusedMaxT && L->chunk_ws &&
        gdn::delta_chunked_workspace(r.B, r.T, d.num_v_heads, d.head_k_dim, d.head_v_dim) <= L->chunk_ws_bytes)
        return gdn::launch_delta_chunked(r, d.head_k_dim, d.head_v_dim, L->chunk_ws, L->chunk_ws_bytes, st);
    return gdn::launch_delta_seq(r, d.head_k_dim, d.head_v_dim, st);
}

int run_chunk(gdn_layer* L, const u16* x, int B, int T, const int* slot_ids, u16* out, hipStream_t st) {
    const gdn_dims& d = L->d;
    const int M = B * T;
    hipEvent_t ev[4] = {L->prof_event(0), L->prof_event(1), L->prof_event(2), L->prof_event(3)};
    if (ev[0]) HIP_OK(hipEventRecord(ev[0], st));
    // decode-sized launches stream the weights against fragment-tiled activations
    const bool frag = M <= 64;
    const bool y_frag = frag && T <= kFusedMaxT;  // the fused mixer writes y straight into W_FRAG layout
    if (frag) HIP_OK(gdn::launch_frag_tile(x, M, d.hidden, L->x_frag, st));
    HIP_OK(gdn::launch_linear(frag ? L->x_frag : x, frag ? gdn::W_FRAG : gdn::W_ROW, L->w_in, gdn::W_FRAG, M, L->NP,
                              d.hidden, L->P, gdn::OUT_F32, st));
    if (ev[1]) HIP_OK(hipEventRecord(ev[1], st));
    if (T <= kFusedMaxT) {
        gdn::MixerArgs a{};
        a.P = L->P, a.NP = L->NP, a.B = B, a.T = T, a.slot_ids = slot_ids;
        a.nk = d.num_k_heads, a.nv = d.num_v_heads;
        a.conv_w = L->conv_w, a.neg_A = L->neg_A, a.dt_bias = L->dt_bias, a.norm_w = L->norm_w;
        a.eps = d.rms_norm_eps;
        a.rec_state = L->rec, a.conv_state = L->conv;
        a.y = L->y, a.y_frag = y_frag ? 1 : 0, a.o_tap = nullptr;
        HIP_OK(gdn::launch_mixer(a, d.head_k_dim, d.head_v_dim, st));
    } else {
        gdn::FrontArgs f{};
        f.P = L->P, f.NP = L->NP, f.B = B, f.T = T, f.slot_ids = slot_ids;
        f.nk = d.num_k_heads, f.nv = d.num_v_heads, f.dk = d.head_k_dim, f.dv = d.head_v_dim;
        f.conv_w = L->conv_w, f.neg_A = L->neg_A, f.dt_bias = L->dt_bias;
        f.conv_state = L->conv;
        f.qn = L->qn, f.kn = L->kn, f.v = L->v, f.g = L->g, f.beta = L->beta;
        HIP_OK(gdn::launch_conv_front(f, st));
        HIP_OK(gdn::launch_conv_commit(L->P, L->NP, B, T, slot_ids, d.num_k_heads, d.num_v_heads, d.head_k_dim,
                                       d.head_v_dim, L->conv, st));
        gdn::DeltaArgs r{};
        r.q = L->qn, r.k = L->kn, r.v = L->v, r.g = L->g, r.beta = L->beta;
        r.B = B, r.T = T, r.Hk = d.num_k_heads, r.Hv = d.num_v_heads, r.slot_ids = slot_ids;
        r.state = L->rec, r.o = L->o, r.normalize = 0, r.scale = 1.f;
        HIP_OK(run_delta(L, r, st));
        HIP_OK(gdn::launch_gated_rmsnorm(L->o, M, d.num_v_heads, d.head_v_dim, L->P + L->CD, L->NP, L->norm_w,
                                         d.rms_norm_eps, L->y, st));
    }
    if (ev[2]) HIP_OK(hipEventRecord(ev[2], st));
    HIP_OK(gdn::launch_linear(L->y, y_frag ? gdn::W_FRAG : gdn::W_ROW, L->w_out, gdn::W_FRAG, M, d.hidden, L->Vd, out,
                              gdn::OUT_BF16, st));
    if (ev[3]) {
        HIP_OK(hipEventRecord(ev[3], st));
        ++L->prof_calls;
    }
    return GDN_OK;
}

}  // namespace

extern "C" {

const char* gdn_last_error(void) { return g_last_error.c_str(); }

int gdn_version(void) { return 100; }

int gdn_layer_create(const gdn_dims* dims, const gdn_weights* w, int max_slots, int max_tokens, gdn_layer** out) {
    if (!out) return fail(GDN_ERR_INVALID_ARG, "out is NULL");
    *out = nullptr;
    int rc = check_dims(dims);
    if (rc) return rc;
    if (!w || !w->in_proj_qkv || !w->in_proj_z || !w->in_proj_a || !w->in_proj_b || !w->conv1d || !w->A_log ||
        !w->dt_bias || !w->norm_weight || !w->out_proj)
        return fail(GDN_ERR_INVALID_ARG, "a weight pointer is NULL");
    if (max_slots <= 0 || max_tokens <= 0) return fail(GDN_ERR_INVALID_ARG, "max_slots and max_tokens must be > 0");

    gdn_layer* L = new gdn_layer();
    L->d = *dims;
    const gdn_dims& d = L->d;
    const int H = d.hidden, nk = d.num_k_heads, nv = d.num_v_heads, dk = d.head_k_dim, dv = d.head_v_dim;
    L->Kd = nk * dk, L->Vd = nv * dv, L->CD = 2 * L->Kd + L->Vd, L->NP = L->CD + L->Vd + 2 * nv;
    L->CH = 2 * dk + dv;
    L->max_slots = max_slots, L->max_tokens = max_tokens;
    const size_t MT = (size_t)max_tokens;

    hipError_t e = hipSuccess;
    auto take = [&](hipError_t r) {
        if (e == hipSuccess) e = r;
    };
    take(L->alloc(&L->w_in, gdn::frag_elems(L->NP, H)));
    take(L->alloc(&L->w_out, gdn::frag_elems(H, L->Vd)));
    take(L->alloc(&L->conv_w, (size_t)L->CD));
    take(L->alloc(&L->neg_A, (size_t)nv));
    take(L->alloc(&L->dt_bias, (size_t)nv));
    take(L->alloc(&L->norm_w, (size_t)dv));
    take(L->alloc(&L->rec, (size_t)max_slots * nv * dk * dv));
    take(L->alloc(&L->conv, (size_t)max_slots * nv * 3 * L->CH));
    take(L->alloc(&L->x_ws, MT * H));
    take(L->alloc(&L->x_frag, gdn::frag_elems(64, H)));
    take(L->alloc(&L->out_ws, MT * H));
    take(L->alloc(&L->P, MT * L->NP));
    take(L->alloc(&L->qn, MT * L->Kd));
    take(L->alloc(&L->kn, MT * L->Kd));
    take(L->alloc(&L->v, MT * L->Vd));
    take(L->alloc(&L->g, MT * nv));
    take(L->alloc(&L->beta, MT * nv));
    take(L->alloc(&L->o, MT * L->Vd));
    take(L->alloc(&L->y, std::max(MT * L->Vd, gdn::frag_elems(64, L->Vd))));  // W_FRAG y pads rows to 16
    if (max_tokens > kFusedMaxT && gdn::delta_chunked_supported(dk, dv)) {
        // chunked-prefill workspace for the worst launch: B sequences of T > kFusedMaxT tokens with
        // B * T <= max_tokens hold at most max_tokens / 64 + max_tokens / 65 + 1 chunks
        const int chunks = max_tokens / 64 + max_tokens / (kFusedMaxT + 1) + 1;
        L->chunk_ws_bytes = gdn::delta_chunked_workspace(1, 64 * chunks, nv, dk, dv);
        char* p = nullptr;
        take(L->alloc(&p, L->chunk_ws_bytes));
        L->chunk_ws = p;
    }
    if (e != hipSuccess) {
        delete L;
        return fail(e == hipErrorOutOfMemory ? GDN_ERR_OUT_OF_MEMORY : GDN_ERR_HIP, "gdn_layer_create: %s",
                    hipGetErrorString(e));
    }

    // fused in_proj rows: q | k | v (in_proj_qkv), z, a, b -- one weight stream per token.  The HF
    // row-major weights are staged in a temporary device buffer and re-laid out into fragment blocks.
    const size_t row = (size_t)H * sizeof(u16);
    u16* stage = nullptr;
    e = hipMalloc(&stage, std::max((size_t)L->NP * H, (size_t)H * L->Vd) * sizeof(u16));
    if (e == hipSuccess) e = hipMemcpy(stage, w->in_proj_qkv, L->CD * row, hipMemcpyDefault);
    if (e == hipSuccess) e = hipMemcpy(stage + (size_t)L->CD * H, w->in_proj_z, L->Vd * row, hipMemcpyDefault);
    if (e == hipSuccess) e = hipMemcpy(stage + (size_t)(L->CD + L->Vd) * H, w->in_proj_a, nv * row, hipMemcpyDefault);
    if (e == hipSuccess)
        e = hipMemcpy(stage + (size_t)(L->CD + L->Vd + nv) * H, w->in_proj_b, nv * row, hipMemcpyDefault);
    if (e == hipSuccess) e = gdn::launch_frag_tile(stage, L->NP, H, L->w_in, nullptr);
    if (e == hipSuccess) e = hipMemcpy(stage, w->out_proj, (size_t)H * L->Vd * sizeof(u16), hipMemcpyDefault);
    if (e == hipSuccess) e = gdn::launch_frag_tile(stage, H, L->Vd, L->w_out, nullptr);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (stage) (void)hipFree(stage);
    if (e == hipSuccess) e = hipMemcpy(L->conv_w, w->conv1d, (size_t)L->CD * 4 * sizeof(float), hipMemcpyDefault);
    std::vector<float> host(nv);
    if (e == hipSuccess) e = hipMemcpy(host.data(), w->A_log, nv * sizeof(float), hipMemcpyDefault);
    if (e == hipSuccess) {
        for (float& a : host) a = -std::exp(a);  // g = -exp(A_log) softplus(.)  (9B/gdn_layer.py:125)
        e = hipMemcpy(L->neg_A, host.data(), nv * sizeof(float), hipMemcpyDefault);
    }
    if (e == hipSuccess) e = hipMemcpy(L->dt_bias, w->dt_bias, nv * sizeof(float), hipMemcpyDefault);
    if (e == hipSuccess) e = hipMemcpy(L->norm_w, w->norm_weight, dv * sizeof(float), hipMemcpyDefault);
    if (e == hipSuccess) e = gdn::launch_state_zero(L->rec, L->conv, nullptr, max_slots, nv, dk, dv,
                                                    L->CH, nullptr);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        delete L;
        return fail(GDN_ERR_HIP, "gdn_layer_create: %s", hipGetErrorString(e));
    }
    *out = L;
    return GDN_OK;
}

int gdn_layer_destroy(gdn_layer* L) {
    if (!L) return GDN_OK;
    (void)hipDeviceSynchronize();
    delete L;
    return GDN_OK;
}

int gdn_layer_forward(gdn_layer* L, const void* x, int B, int T, const int* slot_ids, void* out, void* stream) {
    if (!L || !x || !out) return fail(GDN_ERR_INVALID_ARG, "gdn_layer_forward: NULL argument");
    if (B <= 0 || T <= 0) return fail(GDN_ERR_SHAPE, "gdn_layer_forward: B=%d T=%d must be > 0", B, T);
    if (B > L->max_tokens) return fail(GDN_ERR_SHAPE, "B=%d exceeds max_tokens=%d", B, L->max_tokens);
    if (!slot_ids && B > L->max_slots) return fail(GDN_ERR_SLOT, "B=%d exceeds max_slots=%d", B, L->max_slots);
    const hipStream_t st = as_stream(stream);
    const int H = L->d.hidden;
    const int tc_max = L->max_tokens / B;
    if (T <= tc_max) return run_chunk(L, (const u16*)x, B, T, slot_ids, (u16*)out, st);
    for (int t0 = 0; t0 < T; t0 += tc_max) {
        const int tc = T - t0 < tc_max ? T - t0 : tc_max;
        const size_t rb = (size_t)H * sizeof(u16);
        if (B == 1) {
            int rc = run_chunk(L, (const u16*)x + (size_t)t0 * H, 1, tc, slot_ids, (u16*)out + (size_t)t0 * H, st);
            if (rc) return rc;
            continue;
        }
        // gather rows [b, t0:t0+tc) of every sequence into one sequence-major block, and scatter back
        HIP_OK(hipMemcpy2DAsync(L->x_ws, tc * rb, (const u16*)x + (size_t)t0 * H, (size_t)T * rb, tc * rb, B,
                                hipMemcpyDeviceToDevice, st));
        int rc = run_chunk(L, L->x_ws, B, tc, slot_ids, L->out_ws, st);
        if (rc) return rc;
        HIP_OK(hipMemcpy2DAsync((u16*)out + (size_t)t0 * H, (size_t)T * rb, L->out_ws, tc * rb, tc * rb, B,
                                hipMemcpyDeviceToDevice, st));
    }
    return GDN_OK;
}

int gdn_state_reset(gdn_layer* L, const int* slot_ids, int n, void* stream) {
    if (!L) return fail(GDN_ERR_INVALID_ARG, "layer is NULL");
    if (n < 0 || (!slot_ids && n > L->max_slots)) return fail(GDN_ERR_SLOT, "bad slot count %d", n);
    const gdn_dims& d = L->d;
    HIP_OK(gdn::launch_state_zero(L->rec, L->conv, slot_ids, n, d.num_v_heads, d.head_k_dim,
                                  d.head_v_dim, L->CH, as_stream(stream)));
    return GDN_OK;
}

int gdn_state_get(gdn_layer* L, const int* slot_ids, int n, float* rec, float* conv, void* stream) {
    if (!L || (!rec && !conv)) return fail(GDN_ERR_INVALID_ARG, "gdn_state_get: NULL argument");
    if (n < 0 || (!slot_ids && n > L->max_slots)) return fail(GDN_ERR_SLOT, "bad slot count %d", n);
    const gdn_dims& d = L->d;
    HIP_OK(gdn::launch_state_export(L->rec, L->conv, slot_ids, n, d.num_k_heads, d.num_v_heads,
                                    d.head_k_dim, d.head_v_dim, rec, conv, as_stream(stream)));
    return GDN_OK;
}

int gdn_state_set(gdn_layer* L, const int* slot_ids, int n, const float* rec, const float* conv, void* stream) {
    if (!L) return fail(GDN_ERR_INVALID_ARG, "layer is NULL");
    if (n < 0 || (!slot_ids && n > L->max_slots)) return fail(GDN_ERR_SLOT, "bad slot count %d", n);
    const gdn_dims& d = L->d;
    HIP_OK(gdn::launch_state_import(L->rec, L->conv, slot_ids, n, d.num_k_heads, d.num_v_heads,
                                    d.head_k_dim, d.head_v_dim, rec, conv, as_stream(stream)));
    return GDN_OK;
}

int gdn_layer_state_buffers(gdn_layer* L, void** rec, void** conv) {
    if (!L) return fail(GDN_ERR_INVALID_ARG, "layer is NULL");
    if (rec) *rec = L->rec;
    if (conv) *conv = L->conv;
    return GDN_OK;
}

int gdn_layer_profile(gdn_layer* L, int max_calls) {
    if (!L || max_calls < 0) return fail(GDN_ERR_INVALID_ARG, "gdn_layer_profile: bad argument");
    L->prof_free();
    L->prof_events.resize((size_t)max_calls * 4, nullptr);
    for (hipEvent_t& e : L->prof_events) HIP_OK(hipEventCreate(&e));
    L->prof_max = max_calls;
    return GDN_OK;
}

int gdn_layer_profile_read(gdn_layer* L, double* ms, int* calls) {
    if (!L || !ms) return fail(GDN_ERR_INVALID_ARG, "gdn_layer_profile_read: NULL argument");
    for (int i = 0; i < 4; ++i) ms[i] = 0.0;
    if (calls) *calls = L->prof_calls;
    if (L->prof_calls == 0) return GDN_OK;
    HIP_OK(hipEventSynchronize(L->prof_events[(size_t)(L->prof_calls - 1) * 4 + 3]));
    for (int c = 0; c < L->prof_calls; ++c) {
        const hipEvent_t* e = &L->prof_events[(size_t)c * 4];
        for (int s = 0; s < 3; ++s) {
            float t = 0.f;
            HIP_OK(hipEventElapsedTime(&t, e[s], e[s + 1]));
            ms[s] += t;
        }
        float t = 0.f;
        HIP_OK(hipEventElapsedTime(&t, e[0], e[3]));
        ms[3] += t;
    }
    return GDN_OK;
}

int gdn_layer_proj_width(const gdn_layer* L) { return L ? L->NP : fail(GDN_ERR_INVALID_ARG, "layer is NULL"); }

int gdn_in_proj(gdn_layer* L, const void* x, int M, float* P, void* stream) {
    if (!L || !x || !P) return fail(GDN_ERR_INVALID_ARG, "gdn_in_proj: NULL argument");
    if (M <= 0) return fail(GDN_ERR_SHAPE, "M=%d", M);
    HIP_OK(gdn::launch_linear(x, gdn::W_ROW, L->w_in, gdn::W_FRAG, M, L->NP, L->d.hidden, P, gdn::OUT_F32,
                              as_stream(stream)));
    return GDN_OK;
}

int gdn_conv_front(gdn_layer* L, const float* P, int B, int T, const int* slot_ids, float* qn, float* kn, float* v,
                   float* g, float* beta, void* stream) {
    if (!L || !P || !qn || !kn || !v || !g || !beta) return fail(GDN_ERR_INVALID_ARG, "gdn_conv_front: NULL argument");
    if (B <= 0 || T <= 0) return fail(GDN_ERR_SHAPE, "B=%d T=%d", B, T);
    if (!slot_ids && B > L->max_slots) return fail(GDN_ERR_SLOT, "B=%d exceeds max_slots=%d", B, L->max_slots);
    const gdn_dims& d = L->d;
    const hipStream_t st = as_stream(stream);
    gdn::FrontArgs f{};
    f.P = P, f.NP = L->NP, f.B = B, f.T = T, f.slot_ids = slot_ids;
    f.nk = d.num_k_heads, f.nv = d.num_v_heads, f.dk = d.head_k_dim, f.dv = d.head_v_dim;
    f.conv_w = L->conv_w, f.neg_A = L->neg_A, f.dt_bias = L->dt_bias;
    f.conv_state = L->conv;
    f.qn = qn, f.kn = kn, f.v = v, f.g = g, f.beta = beta;
    HIP_OK(gdn::launch_conv_front(f, st));
    HIP_OK(gdn::launch_conv_commit(P, L->NP, B, T, slot_ids, d.num_k_heads, d.num_v_heads, d.head_k_dim,
                                   d.head_v_dim, L->conv, st));
    return GDN_OK;
}

int gdn_delta_rule(gdn_layer* L, const float* qn, const float* kn, const float* v, const float* g, const float* beta,
                   int B, int T, const int* slot_ids, float* o, void* stream) {
    if (!L || !qn || !kn || !v || !g || !beta || !o) return fail(GDN_ERR_INVALID_ARG, "gdn_delta_rule: NULL argument");
    if (B <= 0 || T <= 0) return fail(GDN_ERR_SHAPE, "B=%d T=%d", B, T);
    if (!slot_ids && B > L->max_slots) return fail(GDN_ERR_SLOT, "B=%d exceeds max_slots=%d", B, L->max_slots);
    const gdn_dims& d = L->d;
    gdn::DeltaArgs r{};
    r.q = qn, r.k = kn, r.v = v, r.g = g, r.beta = beta;
    r.B = B, r.T = T, r.Hk = d.num_k_heads, r.Hv = d.num_v_heads, r.slot_ids = slot_ids;
    r.state = L->rec, r.o = o, r.normalize = 0, r.scale = 1.f;
    HIP_OK(run_delta(L, r, as_stream(stream)));
    return GDN_OK;
}

int gdn_gated_rmsnorm(gdn_layer* L, const float* o, const float* z, int z_stride, int M, void* y, void* stream) {
    if (!L || !o || !z || !y) return fail(GDN_ERR_INVALID_ARG, "gdn_gated_rmsnorm: NULL argument");
    if (M <= 0 || z_stride < L->Vd) return fail(GDN_ERR_SHAPE, "M=%d z_stride=%d", M, z_stride);
    const gdn_dims& d = L->d;
    HIP_OK(gdn::launch_gated_rmsnorm(o, M, d.num_v_heads, d.head_v_dim, z, z_stride, L->norm_w, d.rms_norm_eps,
                                     (u16*)y, as_stream(stream)));
    return GDN_OK;
}

int gdn_out_proj(gdn_layer* L, const void* y, int M, void* out, void* stream) {
    if (!L || !y || !out) return fail(GDN_ERR_INVALID_ARG, "gdn_out_proj: NULL argument");
    if (M <= 0) return fail(GDN_ERR_SHAPE, "M=%d", M);
    HIP_OK(gdn::launch_linear(y, gdn::W_ROW, L->w_out, gdn::W_FRAG, M, L->d.hidden, L->Vd, out, gdn::OUT_BF16,
                              as_stream(stream)));
    return GDN_OK;
}

int gdn_delta_rule_fla(const float* q, const float* k, const float* v, const float* g, const float* beta, int B,
                       int T, int Hk, int Hv, int dk, int dv, float* state, int use_qk_l2norm, float scale, float* o,
                       void* stream) {
    if (!q || !k || !v || !g || !beta || !state || !o) return fail(GDN_ERR_INVALID_ARG, "gdn_delta_rule_fla: NULL argument");
    if (B <= 0 || T <= 0 || Hk <= 0 || Hv <= 0) return fail(GDN_ERR_SHAPE, "B=%d T=%d Hk=%d Hv=%d", B, T, Hk, Hv);
    if (Hv % Hk) return fail(GDN_ERR_UNSUPPORTED, "Hv=%d is not a multiple of Hk=%d", Hv, Hk);
    if (dk != dv || !supported_head_dim(dk))
        return fail(GDN_ERR_UNSUPPORTED, "head dims %d x %d: need dk == dv in {32, 64, 128}", dk, dv);
    gdn::DeltaArgs r{};
    r.q = q, r.k = k, r.v = v, r.g = g, r.beta = beta;
    r.B = B, r.T = T, r.Hk = Hk, r.Hv = Hv, r.slot_ids = nullptr;
    r.state = state, r.o = o, r.normalize = use_qk_l2norm ? 1 : 0;
    r.scale = scale > 0.f ? scale : 1.f / std::sqrt((float)dk);
    HIP_OK(gdn::launch_delta_seq(r, dk, dv, as_stream(stream)));
    return GDN_OK;
}

int gdn_linear_bf16(const void* x, const void* w, int M, int N, int K, void* y, int out_fp32, void* stream) {
    if (!x || !w || !y) return fail(GDN_ERR_INVALID_ARG, "gdn_linear_bf16: NULL argument");
    if (M <= 0 || N <= 0 || K <= 0) return fail(GDN_ERR_SHAPE, "M=%d N=%d K=%d", M, N, K);
    if (K % 128) return fail(GDN_ERR_UNSUPPORTED, "K=%d is not a multiple of 128", K);
    HIP_OK(gdn::launch_linear(x, gdn::W_ROW, w, gdn::W_ROW, M, N, K, y, out_fp32 ? gdn::OUT_F32 : gdn::OUT_BF16,
                              as_stream(stream)));
    return GDN_OK;
}

}  // extern "C"

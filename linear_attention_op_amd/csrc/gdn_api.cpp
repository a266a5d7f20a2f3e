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
#include <mutex>
#include <string>
#include <vector>

#include "../../include/gdn.h"
#include "gdn_common.h"

using gdn::u16;
using gdn::u8;

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
// k ranges of the a | b rows in the decode in_proj (the mixer adds the partial sums)
constexpr int kAbSplits = 8;

bool supported_head_dim(int d) { return d == 32 || d == 64 || d == 128; }

}  // namespace

struct gdn_layer {
    gdn_dims d{};
    int Kd = 0, Vd = 0, CD = 0, NP = 0, CH = 0;
    int max_slots = 0, max_tokens = 0;
    std::vector<void*> allocs;

    int wfmt = GDN_WEIGHTS_BF16;
    int out_kind = gdn::OUT_BF16;  // element type of the layer's output (gdn_layer_set_output_dtype)
    u16* w_in = nullptr;      // bf16: [NP, H]  rows q | k | v | z | a | b, W_FRAG layout
    u16* w_out = nullptr;     // bf16: [H, Vd] W_FRAG layout
    u16* w_ab = nullptr;      // [2 nv, H] a | b rows, W_FRAG (bf16: inside w_in)
    u8* w_in8 = nullptr;      // fp8: [CD + Vd, H] rows q | k | v | z, W_F8 layout
    float* s_in = nullptr;    // fp8: per-row scales of w_in8
    u8* w_out8 = nullptr;     // fp8: [H, Vd] W_F8 layout
    float* s_out = nullptr;   // fp8: per-row scales of w_out8
    u8* w_in4 = nullptr;      // mxfp4: [CD + Vd, H] rows q | k | v | z, W_F4 layout
    u8* s_in4 = nullptr;      // mxfp4: E8M0 scale codes of w_in4 (f4_scale_offset order)
    u8* w_out4 = nullptr;     // mxfp4: [H, Vd] W_F4 layout
    u8* s_out4 = nullptr;     // mxfp4: scale codes of w_out4
    u8* w_in_i8 = nullptr;    // mxint8: [CD + Vd, H] rows q | k | v | z, int8 codes in W_I8 layout
    u8* s_in_i8 = nullptr;    // mxint8: E8M0 scale codes of w_in_i8 (f4_scale_offset order)
    u8* w_out_i8 = nullptr;   // mxint8: [H, Vd] W_I8 layout
    u8* s_out_i8 = nullptr;   // mxint8: scale codes of w_out_i8
    float4* conv_w = nullptr; // [CD] taps
    float* neg_A = nullptr;   // [nv]
    float* dt_bias = nullptr; // [nv]
    float* norm_w = nullptr;  // [dv]
    float* rec = nullptr;     // [slots, nv, dk, dv]
    float* conv = nullptr;    // [slots, nk, 4, CH] conv history rings, one per k-head group
    int* conv_pos = nullptr;  // [slots, nv] ring positions, one per v-head

    int* iota = nullptr;      // [max_slots] identity slot ids (slot offsets of varlen groups)

    // workspace, sized for max_tokens rows; layers of a stack share one (run one at a time)
    bool owns_ws = true;
    std::vector<void*> ws_allocs;
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
    float* ab = nullptr;      // [kAbSplits, 64, 2 nv] partial a | b of the decode in_proj
    float* ss = nullptr;      // [kGnormMaxM, nv, kMixerSplit] partial sums of squares of a split-head launch
    void* chunk_ws = nullptr;
    size_t chunk_ws_bytes = 0;

    // stage timing: 4 events per recorded call (start, after in_proj, after mixer, after out_proj)
    std::vector<hipEvent_t> prof_events;
    int prof_max = 0, prof_calls = 0;

    template <typename Tp>
    hipError_t alloc(Tp** p, size_t count, bool workspace = false) {
        void* q = nullptr;
        hipError_t e = hipMalloc(&q, count * sizeof(Tp) > 0 ? count * sizeof(Tp) : 16);
        if (e == hipSuccess) (workspace ? ws_allocs : allocs).push_back(q);
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
        for (void* p : ws_allocs) (void)hipFree(p);
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
    // the fused mixer runs a k-head group (k-head and its v-heads, 256 threads each) in one workgroup
    if (d->num_v_heads / d->num_k_heads > 4)
        return fail(GDN_ERR_UNSUPPORTED, "num_v_heads / num_k_heads = %d (at most 4)", d->num_v_heads / d->num_k_heads);
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

bool fp8(const gdn_layer* L) { return L->wfmt == GDN_WEIGHTS_FP8_E4M3; }
bool fp4(const gdn_layer* L) { return L->wfmt == GDN_WEIGHTS_MXFP4; }
bool int8w(const gdn_layer* L) { return L->wfmt == GDN_WEIGHTS_MXINT8; }
// the q | k | v | z rows of in_proj, and out_proj, as stored: (weights, layout, scales)
struct QW {
    const void* w;
    int layout;
    const float* scale;
};
QW w_in_q(const gdn_layer* L) {
    if (fp8(L)) return {L->w_in8, gdn::W_F8, L->s_in};
    if (fp4(L)) return {L->w_in4, gdn::W_F4, reinterpret_cast<const float*>(L->s_in4)};
    if (int8w(L)) return {L->w_in_i8, gdn::W_I8, reinterpret_cast<const float*>(L->s_in_i8)};
    return {L->w_in, gdn::W_FRAG, nullptr};
}
QW w_out_q(const gdn_layer* L) {
    if (fp8(L)) return {L->w_out8, gdn::W_F8, L->s_out};
    if (fp4(L)) return {L->w_out4, gdn::W_F4, reinterpret_cast<const float*>(L->s_out4)};
    if (int8w(L)) return {L->w_out_i8, gdn::W_I8, reinterpret_cast<const float*>(L->s_out_i8)};
    return {L->w_out, gdn::W_FRAG, nullptr};
}

// in_proj of M rows (x row-major, or W_FRAG for M <= 64) into P [M, NP] (9B/gdn_layer.py:255-259).  FP8
// layers run the q | k | v | z rows on E4M3 weights and the a | b rows on bf16 ones.
// Prefill-sized launches take the q | k | v | z rows (a multiple of 256 at the model shapes, so whole
// 256-wide GEMM tiles) and the a | b rows as two GEMMs: one partial column of 256-wide tiles would cost a
// full round of workgroups for 64 useful columns.
hipError_t in_proj_rows(const gdn_layer* L, const void* x, int xl, int M, float* P, hipStream_t st) {
    const int H = L->d.hidden, N1 = L->CD + L->Vd, nab = 2 * L->d.num_v_heads;
    if (L->wfmt == GDN_WEIGHTS_BF16 && M <= 64)
        return gdn::launch_linear(x, xl, L->w_in, gdn::W_FRAG, nullptr, M, L->NP, H, P, L->NP, gdn::OUT_F32, st);
    const QW q = w_in_q(L);
    hipError_t e = gdn::launch_linear(x, xl, q.w, q.layout, q.scale, M, N1, H, P, L->NP, gdn::OUT_F32, st);
    if (e != hipSuccess) return e;
    // the a | b rows: for prefills the GEMV with the roles swapped (the activations streamed once)
    // (at most 64 weight rows; wider a | b blocks run as an ordinary projection)
    if (M > 64 && nab <= 64) return gdn::launch_linear_rows_t(x, L->w_ab, nab, M, H, P + N1, L->NP, st);
    return gdn::launch_linear(x, xl, L->w_ab, gdn::W_FRAG, nullptr, M, nab, H, P + N1, L->NP, gdn::OUT_F32, st);
}

// out_proj of M rows of y (row-major, or W_FRAG for M <= 64) into out [M, H], bf16 or fp32 by out_kind
// (9B/gdn_layer.py:272-276).  Both kinds store the same fp32 sums; bf16 rounds them to nearest even.
hipError_t out_proj_rows(const gdn_layer* L, const void* y, int yl, int M, void* out, int out_kind,
                         hipStream_t st) {
    const int H = L->d.hidden;
    const QW q = w_out_q(L);
    return gdn::launch_linear(y, yl, q.w, q.layout, q.scale, M, H, L->Vd, out, H, out_kind, st);
}

// bytes of one output element of an out_kind
size_t out_elem_bytes(int out_kind) { return out_kind == gdn::OUT_F32 ? sizeof(float) : sizeof(u16); }

// A group of sequences of one launch with the same length: rows [row0, row0 + B T) of the launch,
// sequence b of the group on state slot slots[b].
struct Group {
    int row0, B, T;
    const int* slots;  // device [B]; never NULL here
};

// One launch over M rows made of row groups (9B/gdn_layer.py:244-280 for a single group): the in_proj over
// all M rows, the middle of the layer per group (fused mixer for groups of <= kFusedMaxT tokens per
// sequence, front end + chunked recurrence + gated RMSNorm otherwise), the out_proj over all M rows.
int run_rows(gdn_layer* L, const u16* x, int M, const Group* grp, int ng, void* out, int out_kind, hipStream_t st) {
    const gdn_dims& d = L->d;
    const int Kd = L->Kd, Vd = L->Vd, nv = d.num_v_heads;
    hipEvent_t ev[4] = {L->prof_event(0), L->prof_event(1), L->prof_event(2), L->prof_event(3)};
    if (ev[0]) HIP_OK(hipEventRecord(ev[0], st));
    // decode-sized launches stream the weights against fragment-tiled activations
    const bool frag = M <= 64;
    // the fused mixer writes y straight into W_FRAG layout when it produces every row
    const bool y_frag = frag && ng == 1 && grp[0].T <= kFusedMaxT;
    // single-token launches of at most 64 (sequence, v-head) pairs would leave most CUs idle with one
    // workgroup per head: each head's state is split over kMixerSplit workgroups, and the gated RMSNorm
    // moves into the out_proj (128-wide heads; bf16 weights need the value width at 2048 or 4096).  Not
    // with MXINT8 weights, whose heavier GEMV gains nothing from it: the 9B batch-1 step took 32.6 against
    // 32.5 us split (33.9 before the out_proj touched its weight lines ahead of the norm).
    const bool split_heads = y_frag && grp[0].T == 1 && M * nv <= 64 && M <= gdn::kGnormMaxM &&
                             d.head_k_dim == 128 && d.head_v_dim == 128 && Vd <= gdn::kGnormMaxK &&
                             L->wfmt != GDN_WEIGHTS_MXINT8 &&
                             (L->wfmt != GDN_WEIGHTS_BF16 || Vd == 4096 || Vd == 2048) && L->NP % 4 == 0;
    // decode: q | k | v | z over workgroups balanced on the CUs, a | b as partial sums for the mixer
    const bool split_ab = frag && gdn::in_proj_decode_supported(L->CD + Vd, L->d.hidden);
    bool ab_split = false;
    if (frag) {
        bool mixer_only = true;
        for (int gi = 0; gi < ng; ++gi) mixer_only = mixer_only && grp[gi].T <= kFusedMaxT;
        ab_split = split_ab && mixer_only;
    }
    // up to 16 rows the decode in_proj reads the activations row-major: re-tiling them would cost a launch
    const bool x_rows = ab_split && M <= 16;
    if (frag && !x_rows) HIP_OK(gdn::launch_frag_tile(x, M, d.hidden, L->x_frag, st));
    if (ab_split) {
        const QW q = w_in_q(L);
        HIP_OK(gdn::launch_in_proj_decode(x_rows ? (const void*)x : L->x_frag, x_rows ? gdn::W_ROW : gdn::W_FRAG,
                                          q.w, q.layout, q.scale, L->w_ab, M, L->CD + Vd, 2 * nv, d.hidden, L->P,
                                          L->NP, L->ab, kAbSplits, st));
    } else
        HIP_OK(in_proj_rows(L, frag ? L->x_frag : x, frag ? gdn::W_FRAG : gdn::W_ROW, M, L->P, st));
    if (ev[1]) HIP_OK(hipEventRecord(ev[1], st));
    for (int gi = 0; gi < ng; ++gi) {
        const Group& g = grp[gi];
        const size_t r0 = (size_t)g.row0;
        const int Mg = g.B * g.T;
        if (g.T <= kFusedMaxT) {
            gdn::MixerArgs a{};
            a.P = L->P + r0 * L->NP, a.NP = L->NP, a.B = g.B, a.T = g.T, a.slot_ids = g.slots;
            a.max_slots = L->max_slots, a.nk = d.num_k_heads, a.nv = nv;
            a.conv_w = L->conv_w, a.neg_A = L->neg_A, a.dt_bias = L->dt_bias, a.norm_w = L->norm_w;
            a.eps = d.rms_norm_eps;
            a.rec_state = L->rec, a.conv_state = L->conv, a.conv_pos = L->conv_pos;
            a.y = y_frag ? L->y : L->y + r0 * Vd, a.y_frag = y_frag ? 1 : 0, a.o_tap = nullptr;
            if (split_heads) a.o_tap = L->o, a.ss_part = L->ss;
            a.ab = ab_split ? L->ab + r0 * 2 * nv : nullptr, a.ab_splits = kAbSplits;
            a.ab_stride = (size_t)M * 2 * nv;
            HIP_OK(gdn::launch_mixer(a, d.head_k_dim, d.head_v_dim, st));
        } else {
            float* P = L->P + r0 * L->NP;
            gdn::FrontArgs f{};
            f.P = P, f.NP = L->NP, f.B = g.B, f.T = g.T, f.slot_ids = g.slots, f.max_slots = L->max_slots;
            f.nk = d.num_k_heads, f.nv = nv, f.dk = d.head_k_dim, f.dv = d.head_v_dim;
            f.conv_w = L->conv_w, f.neg_A = L->neg_A, f.dt_bias = L->dt_bias;
            f.conv_state = L->conv, f.conv_pos = L->conv_pos;
            f.qn = L->qn + r0 * Kd, f.kn = L->kn + r0 * Kd, f.v = L->v + r0 * Vd;
            f.g = L->g + r0 * nv, f.beta = L->beta + r0 * nv;
            gdn::DeltaArgs r{};
            r.q = f.qn, r.k = f.kn, r.v = f.v, r.g = f.g, r.beta = f.beta;
            r.B = g.B, r.T = g.T, r.Hk = d.num_k_heads, r.Hv = nv, r.slot_ids = g.slots;
            r.max_slots = L->max_slots, r.state = L->rec, r.o = L->o + r0 * Vd, r.normalize = 0, r.scale = 1.f;
            if (L->chunk_ws && gdn::delta_chunked_supported(d.head_k_dim, d.head_v_dim) &&
                gdn::delta_chunked_workspace(g.B, g.T, nv, d.head_k_dim, d.head_v_dim) <= L->chunk_ws_bytes) {
                // chunked recurrence with the front end computed inside its chunk preparation
                HIP_OK(gdn::launch_front_chunked(f, L->conv, L->conv_pos, r, L->chunk_ws, L->chunk_ws_bytes, st));
            } else {
                HIP_OK(gdn::launch_conv_front(f, st));
                HIP_OK(gdn::launch_conv_commit(P, L->NP, g.B, g.T, g.slots, L->max_slots, d.num_k_heads, nv,
                                               d.head_k_dim, d.head_v_dim, L->conv, L->conv_pos, st));
                HIP_OK(run_delta(L, r, st));
            }
            HIP_OK(gdn::launch_gated_rmsnorm(r.o, Mg, nv, d.head_v_dim, P + L->CD, L->NP, L->norm_w,
                                             d.rms_norm_eps, L->y + r0 * Vd, st));
        }
    }
    if (ev[2]) HIP_OK(hipEventRecord(ev[2], st));
    if (split_heads) {
        const QW q = w_out_q(L);
        gdn::GnormArgs ga{};
        ga.o = L->o, ga.ss = L->ss, ga.z = L->P + L->CD, ga.ldz = L->NP, ga.norm_w = L->norm_w;
        ga.eps = d.rms_norm_eps, ga.nv = nv, ga.dv = d.head_v_dim;
        ga.w = q.w, ga.scale = q.scale, ga.M = M, ga.N = d.hidden, ga.K = Vd, ga.y = out, ga.ldy = d.hidden;
        ga.conv_pos = L->conv_pos, ga.slot_ids = grp[0].slots, ga.max_slots = L->max_slots;
        HIP_OK(gdn::launch_out_proj_gnorm(ga, q.layout, out_kind, st));
    } else {
        HIP_OK(out_proj_rows(L, L->y, y_frag ? gdn::W_FRAG : gdn::W_ROW, M, out, out_kind, st));
    }
    if (ev[3]) {
        HIP_OK(hipEventRecord(ev[3], st));
        ++L->prof_calls;
    }
    return GDN_OK;
}

int run_chunk(gdn_layer* L, const u16* x, int B, int T, const int* slot_ids, void* out, int out_kind,
              hipStream_t st) {
    const Group g{0, B, T, slot_ids ? slot_ids : L->iota};
    return run_rows(L, x, B * T, &g, 1, out, out_kind, st);
}

// Where the output rows of a split launch over several sequences are gathered before they are scattered to
// their sequences: the bf16 output workspace, or for fp32 rows the projection workspace P ([max_tokens, NP]
// fp32), which the out_proj neither reads nor is followed by a reader of; NULL when P rows are narrower
// than the hidden size.
void* split_out_stage(gdn_layer* L, int out_kind) {
    if (out_kind != gdn::OUT_F32) return L->out_ws;
    return L->NP >= L->d.hidden ? (void*)L->P : nullptr;
}

// gdn_layer_forward without the argument checks: launches longer than the workspace are split by tokens.
int layer_forward(gdn_layer* L, const u16* x, int B, int T, const int* slot_ids, void* out, int out_kind,
                  hipStream_t st) {
    const int H = L->d.hidden;
    const int tc_max = L->max_tokens / B;
    if (T <= tc_max) return run_chunk(L, x, B, T, slot_ids, out, out_kind, st);
    char* o = (char*)out;
    const size_t rb = (size_t)H * sizeof(u16), ob = (size_t)H * out_elem_bytes(out_kind);
    void* stage = split_out_stage(L, out_kind);
    if (B > 1 && !stage)
        return fail(GDN_ERR_UNSUPPORTED, "fp32 output of a split launch of %d sequences needs proj width %d >= "
                    "hidden %d", B, L->NP, H);
    for (int t0 = 0; t0 < T; t0 += tc_max) {
        const int tc = T - t0 < tc_max ? T - t0 : tc_max;
        if (B == 1) {
            int rc = run_chunk(L, x + (size_t)t0 * H, 1, tc, slot_ids, o + (size_t)t0 * ob, out_kind, st);
            if (rc) return rc;
            continue;
        }
        // gather rows [b, t0:t0+tc) of every sequence into one sequence-major block, and scatter back
        HIP_OK(hipMemcpy2DAsync(L->x_ws, tc * rb, x + (size_t)t0 * H, (size_t)T * rb, tc * rb, B,
                                hipMemcpyDeviceToDevice, st));
        int rc = run_chunk(L, L->x_ws, B, tc, slot_ids, stage, out_kind, st);
        if (rc) return rc;
        HIP_OK(hipMemcpy2DAsync(o + (size_t)t0 * ob, (size_t)T * ob, stage, tc * ob, tc * ob, B,
                                hipMemcpyDeviceToDevice, st));
    }
    return GDN_OK;
}

// Row groups of a varlen launch: runs of consecutive sequences with equal length.
int varlen_groups(const gdn_layer* L, int n_seqs, const int* cu, const int* slot_ids, std::vector<Group>* out) {
    out->clear();
    if (n_seqs <= 0 || !cu) return fail(GDN_ERR_INVALID_ARG, "varlen: n_seqs=%d, cu_seqlens %p", n_seqs, (const void*)cu);
    if (cu[0] != 0) return fail(GDN_ERR_SHAPE, "varlen: cu_seqlens[0]=%d must be 0", cu[0]);
    if (!slot_ids && n_seqs > L->max_slots) return fail(GDN_ERR_SLOT, "%d sequences exceed max_slots=%d", n_seqs, L->max_slots);
    for (int i = 0; i < n_seqs;) {
        const int T = cu[i + 1] - cu[i];
        if (T <= 0) return fail(GDN_ERR_SHAPE, "varlen: sequence %d has length %d", i, T);
        int j = i + 1;
        while (j < n_seqs && cu[j + 1] - cu[j] == T) ++j;
        out->push_back(Group{cu[i], j - i, T, (slot_ids ? slot_ids : L->iota) + i});
        i = j;
    }
    if (cu[n_seqs] > L->max_tokens)
        return fail(GDN_ERR_SHAPE, "varlen: %d rows exceed max_tokens=%d", cu[n_seqs], L->max_tokens);
    return GDN_OK;
}

}  // namespace

extern "C" {

const char* gdn_last_error(void) { return g_last_error.c_str(); }

int gdn_version(void) { return 100; }

}  // extern "C"

namespace {

// Layer creation; `share` (a layer of the same geometry) lends its launch workspace, as layers of a stack
// run one at a time.
int create_layer(const gdn_dims* dims, const gdn_weights* w, int max_slots, int max_tokens, int wfmt,
                 const gdn_layer* share, gdn_layer** out) {
    if (!out) return fail(GDN_ERR_INVALID_ARG, "out is NULL");
    *out = nullptr;
    int rc = check_dims(dims);
    if (rc) return rc;
    if (wfmt != GDN_WEIGHTS_BF16 && wfmt != GDN_WEIGHTS_FP8_E4M3 && wfmt != GDN_WEIGHTS_MXFP4 &&
        wfmt != GDN_WEIGHTS_MXINT8)
        return fail(GDN_ERR_INVALID_ARG, "unknown weight format %d", wfmt);
    if (!w || !w->in_proj_qkv || !w->in_proj_z || !w->in_proj_a || !w->in_proj_b || !w->conv1d || !w->A_log ||
        !w->dt_bias || !w->norm_weight || !w->out_proj)
        return fail(GDN_ERR_INVALID_ARG, "a weight pointer is NULL");
    if (max_slots <= 0 || max_tokens <= 0) return fail(GDN_ERR_INVALID_ARG, "max_slots and max_tokens must be > 0");

    gdn_layer* L = new gdn_layer();
    L->d = *dims;
    const gdn_dims& d = L->d;
    const int H = d.hidden, nk = d.num_k_heads, nv = d.num_v_heads, dk = d.head_k_dim, dv = d.head_v_dim;
    L->Kd = nk * dk, L->Vd = nv * dv, L->CD = 2 * L->Kd + L->Vd, L->NP = L->CD + L->Vd + 2 * nv;
    L->CH = gdn::conv_group_width(dk, dv, nv / nk);
    L->max_slots = max_slots, L->max_tokens = max_tokens;
    L->wfmt = wfmt;
    const size_t MT = (size_t)max_tokens;
    const int N1 = L->CD + L->Vd;  // q | k | v | z rows (a multiple of 16)

    hipError_t e = hipSuccess;
    auto take = [&](hipError_t r) {
        if (e == hipSuccess) e = r;
    };
    if (wfmt == GDN_WEIGHTS_FP8_E4M3) {
        take(L->alloc(&L->w_in8, gdn::frag_elems(N1, H)));
        take(L->alloc(&L->s_in, (size_t)N1));
        take(L->alloc(&L->w_ab, gdn::frag_elems(2 * nv, H)));
        take(L->alloc(&L->w_out8, gdn::frag_elems(H, L->Vd)));
        take(L->alloc(&L->s_out, (size_t)H));
    } else if (wfmt == GDN_WEIGHTS_MXFP4) {
        // codes: half a byte per weight; scales: a byte per 32 (rows padded to 16)
        take(L->alloc(&L->w_in4, gdn::frag_elems(N1, H) / 2));
        take(L->alloc(&L->s_in4, gdn::frag_elems(N1, H) / 32));
        take(L->alloc(&L->w_ab, gdn::frag_elems(2 * nv, H)));
        take(L->alloc(&L->w_out4, gdn::frag_elems(H, L->Vd) / 2));
        take(L->alloc(&L->s_out4, gdn::frag_elems(H, L->Vd) / 32));
    } else if (wfmt == GDN_WEIGHTS_MXINT8) {
        // codes: a byte per weight; scales: a byte per 32 (rows padded to 16)
        take(L->alloc(&L->w_in_i8, gdn::frag_elems(N1, H)));
        take(L->alloc(&L->s_in_i8, gdn::frag_elems(N1, H) / 32));
        take(L->alloc(&L->w_ab, gdn::frag_elems(2 * nv, H)));
        take(L->alloc(&L->w_out_i8, gdn::frag_elems(H, L->Vd)));
        take(L->alloc(&L->s_out_i8, gdn::frag_elems(H, L->Vd) / 32));
    } else {
        take(L->alloc(&L->w_in, gdn::frag_elems(L->NP, H)));
        take(L->alloc(&L->w_out, gdn::frag_elems(H, L->Vd)));
        if (e == hipSuccess) L->w_ab = L->w_in + gdn::frag_elems(N1, H);
    }
    take(L->alloc(&L->conv_w, (size_t)L->CD));
    take(L->alloc(&L->neg_A, (size_t)nv));
    take(L->alloc(&L->dt_bias, (size_t)nv));
    take(L->alloc(&L->norm_w, (size_t)dv));
    take(L->alloc(&L->rec, (size_t)max_slots * nv * dk * dv));
    take(L->alloc(&L->conv, (size_t)max_slots * nk * gdn::CONV_RING * L->CH));
    take(L->alloc(&L->conv_pos, (size_t)max_slots * nv));
    take(L->alloc(&L->iota, (size_t)max_slots));
    if (share) {
        L->owns_ws = false;
        L->x_ws = share->x_ws, L->x_frag = share->x_frag, L->out_ws = share->out_ws, L->P = share->P;
        L->qn = share->qn, L->kn = share->kn, L->v = share->v, L->g = share->g, L->beta = share->beta;
        L->o = share->o, L->y = share->y, L->chunk_ws = share->chunk_ws, L->chunk_ws_bytes = share->chunk_ws_bytes;
        L->ab = share->ab, L->ss = share->ss;
    } else {
        take(L->alloc(&L->x_ws, MT * H, true));
        take(L->alloc(&L->x_frag, gdn::frag_elems(64, H), true));
        take(L->alloc(&L->out_ws, MT * H, true));
        take(L->alloc(&L->P, MT * L->NP, true));
        take(L->alloc(&L->qn, MT * L->Kd, true));
        take(L->alloc(&L->kn, MT * L->Kd, true));
        take(L->alloc(&L->v, MT * L->Vd, true));
        take(L->alloc(&L->g, MT * nv, true));
        take(L->alloc(&L->beta, MT * nv, true));
        take(L->alloc(&L->o, MT * L->Vd, true));
        take(L->alloc(&L->y, std::max(MT * L->Vd, gdn::frag_elems(64, L->Vd)), true));  // W_FRAG y pads rows to 16
        take(L->alloc(&L->ab, (size_t)kAbSplits * 64 * 2 * nv, true));
        take(L->alloc(&L->ss, (size_t)gdn::kGnormMaxM * nv * gdn::kMixerSplit, true));
        if (max_tokens > kFusedMaxT && gdn::delta_chunked_supported(dk, dv)) {
            // chunked-prefill workspace for the worst launch: sequences of T > kFusedMaxT tokens with
            // at most max_tokens rows in all hold at most max_tokens / 64 + max_tokens / 65 + 1 chunks
            const int chunks = max_tokens / 64 + max_tokens / (kFusedMaxT + 1) + 1;
            L->chunk_ws_bytes = gdn::delta_chunked_workspace(1, 64 * chunks, nv, dk, dv);
            char* p = nullptr;
            take(L->alloc(&p, L->chunk_ws_bytes, true));
            L->chunk_ws = p;
        }
    }
    if (e != hipSuccess) {
        delete L;
        return fail(e == hipErrorOutOfMemory ? GDN_ERR_OUT_OF_MEMORY : GDN_ERR_HIP, "gdn_layer_create: %s",
                    hipGetErrorString(e));
    }

    // fused in_proj rows: q | k | v (in_proj_qkv), z, a, b -- one weight stream per token.  The HF
    // row-major weights are staged in a temporary device buffer and re-laid out into fragment blocks
    // (FP8 / MXFP4 / MXINT8: the q | k | v | z rows and out_proj quantized to E4M3 with per-row scales, to MXFP4
    // or to MXINT8, as
    // the reference converts w_in and w_out to its weight_dtype and keeps w_ab bf16, 9B/gdn_layer.py:115-120).
    const size_t row = (size_t)H * sizeof(u16);
    u16* stage = nullptr;
    e = hipMalloc(&stage, std::max((size_t)L->NP * H, (size_t)H * L->Vd) * sizeof(u16));
    if (e == hipSuccess) e = hipMemcpy(stage, w->in_proj_qkv, L->CD * row, hipMemcpyDefault);
    if (e == hipSuccess) e = hipMemcpy(stage + (size_t)L->CD * H, w->in_proj_z, L->Vd * row, hipMemcpyDefault);
    if (e == hipSuccess) e = hipMemcpy(stage + (size_t)(L->CD + L->Vd) * H, w->in_proj_a, nv * row, hipMemcpyDefault);
    if (e == hipSuccess)
        e = hipMemcpy(stage + (size_t)(L->CD + L->Vd + nv) * H, w->in_proj_b, nv * row, hipMemcpyDefault);
    if (e == hipSuccess) {
        if (wfmt == GDN_WEIGHTS_FP8_E4M3) {
            e = gdn::launch_quantize_e4m3(stage, N1, H, L->w_in8, L->s_in, 1, nullptr);
            if (e == hipSuccess) e = gdn::launch_frag_tile(stage + (size_t)N1 * H, 2 * nv, H, L->w_ab, nullptr);
        } else if (wfmt == GDN_WEIGHTS_MXFP4) {
            e = gdn::launch_quantize_mxfp4(stage, N1, H, L->w_in4, L->s_in4, 1, nullptr);
            if (e == hipSuccess) e = gdn::launch_frag_tile(stage + (size_t)N1 * H, 2 * nv, H, L->w_ab, nullptr);
        } else if (wfmt == GDN_WEIGHTS_MXINT8) {
            e = gdn::launch_quantize_mxint8(stage, N1, H, L->w_in_i8, L->s_in_i8, 1, nullptr);
            if (e == hipSuccess) e = gdn::launch_frag_tile(stage + (size_t)N1 * H, 2 * nv, H, L->w_ab, nullptr);
        } else {
            e = gdn::launch_frag_tile(stage, L->NP, H, L->w_in, nullptr);
        }
    }
    // the stage is reused: finish reading it first
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipMemcpy(stage, w->out_proj, (size_t)H * L->Vd * sizeof(u16), hipMemcpyDefault);
    if (e == hipSuccess) {
        if (wfmt == GDN_WEIGHTS_FP8_E4M3)
            e = gdn::launch_quantize_e4m3(stage, H, L->Vd, L->w_out8, L->s_out, 1, nullptr);
        else if (wfmt == GDN_WEIGHTS_MXFP4)
            e = gdn::launch_quantize_mxfp4(stage, H, L->Vd, L->w_out4, L->s_out4, 1, nullptr);
        else if (wfmt == GDN_WEIGHTS_MXINT8)
            e = gdn::launch_quantize_mxint8(stage, H, L->Vd, L->w_out_i8, L->s_out_i8, 1, nullptr);
        else
            e = gdn::launch_frag_tile(stage, H, L->Vd, L->w_out, nullptr);
    }
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
    if (e == hipSuccess) {
        std::vector<int> ids(max_slots);
        for (int i = 0; i < max_slots; ++i) ids[i] = i;
        e = hipMemcpy(L->iota, ids.data(), max_slots * sizeof(int), hipMemcpyHostToDevice);
    }
    if (e == hipSuccess) e = gdn::launch_state_zero(L->rec, L->conv, L->conv_pos, nullptr, max_slots, max_slots, nk,
                                                    nv, dk, dv, nullptr);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        delete L;
        return fail(GDN_ERR_HIP, "gdn_layer_create: %s", hipGetErrorString(e));
    }
    *out = L;
    return GDN_OK;
}

}  // namespace

extern "C" {

int gdn_layer_create(const gdn_dims* dims, const gdn_weights* w, int max_slots, int max_tokens, gdn_layer** out) {
    return create_layer(dims, w, max_slots, max_tokens, GDN_WEIGHTS_BF16, nullptr, out);
}

int gdn_layer_create_ex(const gdn_dims* dims, const gdn_weights* w, int max_slots, int max_tokens,
                        int weight_format, gdn_layer** out) {
    return create_layer(dims, w, max_slots, max_tokens, weight_format, nullptr, out);
}

int gdn_layer_weight_format(const gdn_layer* L) { return L ? L->wfmt : fail(GDN_ERR_INVALID_ARG, "layer is NULL"); }

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
    return layer_forward(L, (const u16*)x, B, T, slot_ids, out, L->out_kind, as_stream(stream));
}

int gdn_layer_forward_varlen(gdn_layer* L, const void* x, int n_seqs, const int* cu_seqlens, const int* slot_ids,
                             void* out, void* stream) {
    if (!L || !x || !out) return fail(GDN_ERR_INVALID_ARG, "gdn_layer_forward_varlen: NULL argument");
    std::vector<Group> groups;
    int rc = varlen_groups(L, n_seqs, cu_seqlens, slot_ids, &groups);
    if (rc) return rc;
    return run_rows(L, (const u16*)x, cu_seqlens[n_seqs], groups.data(), (int)groups.size(), out, L->out_kind,
                    as_stream(stream));
}

int gdn_layer_set_output_dtype(gdn_layer* L, int out_dtype) {
    if (!L) return fail(GDN_ERR_INVALID_ARG, "layer is NULL");
    if (out_dtype != GDN_OUT_BF16 && out_dtype != GDN_OUT_FP32)
        return fail(GDN_ERR_INVALID_ARG, "output dtype %d (GDN_OUT_BF16 = 0 or GDN_OUT_FP32 = 1)", out_dtype);
    L->out_kind = out_dtype == GDN_OUT_FP32 ? gdn::OUT_F32 : gdn::OUT_BF16;
    return GDN_OK;
}

int gdn_layer_output_dtype(const gdn_layer* L) {
    if (!L) return fail(GDN_ERR_INVALID_ARG, "layer is NULL");
    return L->out_kind == gdn::OUT_F32 ? GDN_OUT_FP32 : GDN_OUT_BF16;
}

int gdn_state_reset(gdn_layer* L, const int* slot_ids, int n, void* stream) {
    if (!L) return fail(GDN_ERR_INVALID_ARG, "layer is NULL");
    if (n < 0 || (!slot_ids && n > L->max_slots)) return fail(GDN_ERR_SLOT, "bad slot count %d", n);
    const gdn_dims& d = L->d;
    HIP_OK(gdn::launch_state_zero(L->rec, L->conv, L->conv_pos, slot_ids, n, L->max_slots, d.num_k_heads,
                                  d.num_v_heads, d.head_k_dim, d.head_v_dim, as_stream(stream)));
    return GDN_OK;
}

int gdn_state_get(gdn_layer* L, const int* slot_ids, int n, float* rec, float* conv, void* stream) {
    if (!L || (!rec && !conv)) return fail(GDN_ERR_INVALID_ARG, "gdn_state_get: NULL argument");
    if (n < 0 || (!slot_ids && n > L->max_slots)) return fail(GDN_ERR_SLOT, "bad slot count %d", n);
    const gdn_dims& d = L->d;
    HIP_OK(gdn::launch_state_export(L->rec, L->conv, L->conv_pos, slot_ids, n, L->max_slots, d.num_k_heads,
                                    d.num_v_heads, d.head_k_dim, d.head_v_dim, rec, conv, as_stream(stream)));
    return GDN_OK;
}

int gdn_state_set(gdn_layer* L, const int* slot_ids, int n, const float* rec, const float* conv, void* stream) {
    if (!L) return fail(GDN_ERR_INVALID_ARG, "layer is NULL");
    if (n < 0 || (!slot_ids && n > L->max_slots)) return fail(GDN_ERR_SLOT, "bad slot count %d", n);
    const gdn_dims& d = L->d;
    HIP_OK(gdn::launch_state_import(L->rec, L->conv, L->conv_pos, slot_ids, n, L->max_slots, d.num_k_heads,
                                    d.num_v_heads, d.head_k_dim, d.head_v_dim, rec, conv, as_stream(stream)));
    return GDN_OK;
}

int gdn_layer_state_buffers(gdn_layer* L, void** rec, void** conv, void** conv_pos) {
    if (!L) return fail(GDN_ERR_INVALID_ARG, "layer is NULL");
    if (rec) *rec = L->rec;
    if (conv) *conv = L->conv;
    if (conv_pos) *conv_pos = L->conv_pos;
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
    HIP_OK(in_proj_rows(L, x, gdn::W_ROW, M, P, as_stream(stream)));
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
    f.P = P, f.NP = L->NP, f.B = B, f.T = T, f.slot_ids = slot_ids, f.max_slots = L->max_slots;
    f.nk = d.num_k_heads, f.nv = d.num_v_heads, f.dk = d.head_k_dim, f.dv = d.head_v_dim;
    f.conv_w = L->conv_w, f.neg_A = L->neg_A, f.dt_bias = L->dt_bias;
    f.conv_state = L->conv, f.conv_pos = L->conv_pos;
    f.qn = qn, f.kn = kn, f.v = v, f.g = g, f.beta = beta;
    HIP_OK(gdn::launch_conv_front(f, st));
    HIP_OK(gdn::launch_conv_commit(P, L->NP, B, T, slot_ids, L->max_slots, d.num_k_heads, d.num_v_heads,
                                   d.head_k_dim, d.head_v_dim, L->conv, L->conv_pos, st));
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
    r.max_slots = L->max_slots, r.state = L->rec, r.o = o, r.normalize = 0, r.scale = 1.f;
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
    HIP_OK(out_proj_rows(L, y, gdn::W_ROW, M, out, L->out_kind, as_stream(stream)));
    return GDN_OK;
}

int gdn_delta_rule_fla(const float* q, const float* k, const float* v, const float* g, const float* beta, int B,
                       int T, int Hk, int Hv, int dk, int dv, float* state, int use_qk_l2norm, float scale, float* o,
                       void* stream) {
    return gdn_delta_rule_fla_ws(q, k, v, g, beta, B, T, Hk, Hv, dk, dv, state, use_qk_l2norm, scale, o, nullptr, 0,
                                 stream);
}

size_t gdn_delta_rule_fla_workspace_size(int B, int T, int Hv, int dk, int dv) {
    if (B <= 0 || T <= kFusedMaxT || Hv <= 0 || !gdn::delta_chunked_supported(dk, dv)) return 0;
    return gdn::delta_chunked_workspace(B, T, Hv, dk, dv);
}

int gdn_delta_rule_fla_ws(const float* q, const float* k, const float* v, const float* g, const float* beta, int B,
                          int T, int Hk, int Hv, int dk, int dv, float* state, int use_qk_l2norm, float scale,
                          float* o, void* workspace, size_t workspace_bytes, void* stream) {
    if (!q || !k || !v || !g || !beta || !state || !o) return fail(GDN_ERR_INVALID_ARG, "gdn_delta_rule_fla: NULL argument");
    if (B <= 0 || T <= 0 || Hk <= 0 || Hv <= 0) return fail(GDN_ERR_SHAPE, "B=%d T=%d Hk=%d Hv=%d", B, T, Hk, Hv);
    if (Hv % Hk) return fail(GDN_ERR_UNSUPPORTED, "Hv=%d is not a multiple of Hk=%d", Hv, Hk);
    if (dk != dv || !supported_head_dim(dk))
        return fail(GDN_ERR_UNSUPPORTED, "head dims %d x %d: need dk == dv in {32, 64, 128}", dk, dv);
    const size_t need = gdn_delta_rule_fla_workspace_size(B, T, Hv, dk, dv);
    if (workspace && workspace_bytes < need)
        return fail(GDN_ERR_SHAPE, "workspace of %zu bytes, this launch needs %zu", workspace_bytes, need);
    gdn::DeltaArgs r{};
    r.q = q, r.k = k, r.v = v, r.g = g, r.beta = beta;
    r.B = B, r.T = T, r.Hk = Hk, r.Hv = Hv, r.slot_ids = nullptr, r.max_slots = B;
    r.state = state, r.o = o, r.normalize = use_qk_l2norm ? 1 : 0;
    r.scale = scale > 0.f ? scale : 1.f / std::sqrt((float)dk);
    if (workspace && need > 0)
        HIP_OK(gdn::launch_delta_chunked(r, dk, dv, workspace, workspace_bytes, as_stream(stream)));
    else
        HIP_OK(gdn::launch_delta_seq(r, dk, dv, as_stream(stream)));
    return GDN_OK;
}

}  // extern "C"

// ------------------------------------------------------------------------------------------------
// gdn_delta_rule_fla_noalloc: gdn_delta_rule_fla_ws with the chunk workspace in a static device array, for
// callers that cannot allocate.  Each device that runs it holds its own copy of the array until the process
// ends; host code uses the copy's device address from hipGetSymbolAddress, taken once per device.
// ------------------------------------------------------------------------------------------------
namespace {

__device__ __align__(256) unsigned char scratch[GDN_NOALLOC_SCRATCH_BYTES];

std::mutex g_scratch_mu;
std::vector<void*> g_scratch_addr;  // per device: the address of that device's `scratch`

// The address of the current device's scratch array (looked up on the first call on that device).
int scratch_address(void** out) {
    int dev = 0;
    HIP_OK(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if ((size_t)dev >= g_scratch_addr.size()) g_scratch_addr.resize((size_t)dev + 1, nullptr);
    if (!g_scratch_addr[dev]) {
        void* p = nullptr;
        HIP_OK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) return fail(GDN_ERR_HIP, "hipGetSymbolAddress returned no address for the scratch array");
        g_scratch_addr[dev] = p;
    }
    *out = g_scratch_addr[dev];
    return GDN_OK;
}

}  // namespace

extern "C" {

int gdn_delta_rule_fla_noalloc(const float* q, const float* k, const float* v, const float* g, const float* beta,
                               int B, int T, int Hk, int Hv, int dk, int dv, float* state, int use_qk_l2norm,
                               float scale, float* o, void* stream) {
    if (B <= 0 || T <= 0 || Hv <= 0)
        return fail(GDN_ERR_SHAPE, "gdn_delta_rule_fla_noalloc: B=%d T=%d Hv=%d", B, T, Hv);
    const size_t need = gdn_delta_rule_fla_workspace_size(B, T, Hv, dk, dv);
    if (need > GDN_NOALLOC_SCRATCH_BYTES)
        return fail(GDN_ERR_SHAPE,
                    "gdn_delta_rule_fla_noalloc: this launch needs %zu bytes of chunk workspace, more than the "
                    "%zu-byte static scratch array (B * Hv * ceil(T / 64) must be at most %zu)",
                    need, (size_t)GDN_NOALLOC_SCRATCH_BYTES,
                    (size_t)GDN_NOALLOC_SCRATCH_BYTES / gdn::delta_chunked_workspace(1, 64, 1, 128, 128));
    void* ws = nullptr;
    if (need > 0) {
        int rc = scratch_address(&ws);
        if (rc) return rc;
    }
    return gdn_delta_rule_fla_ws(q, k, v, g, beta, B, T, Hk, Hv, dk, dv, state, use_qk_l2norm, scale, o, ws,
                                 need > 0 ? (size_t)GDN_NOALLOC_SCRATCH_BYTES : 0, stream);
}

int gdn_linear_bf16(const void* x, const void* w, int M, int N, int K, void* y, int out_fp32, void* stream) {
    if (!x || !w || !y) return fail(GDN_ERR_INVALID_ARG, "gdn_linear_bf16: NULL argument");
    if (M <= 0 || N <= 0 || K <= 0) return fail(GDN_ERR_SHAPE, "M=%d N=%d K=%d", M, N, K);
    if (K % 128) return fail(GDN_ERR_UNSUPPORTED, "K=%d is not a multiple of 128", K);
    HIP_OK(gdn::launch_linear(x, gdn::W_ROW, w, gdn::W_ROW, nullptr, M, N, K, y, N,
                              out_fp32 ? gdn::OUT_F32 : gdn::OUT_BF16, as_stream(stream)));
    return GDN_OK;
}

int gdn_quantize_fp8(const void* w, int N, int K, void* q, float* scale, void* stream) {
    if (!w || !q || !scale) return fail(GDN_ERR_INVALID_ARG, "gdn_quantize_fp8: NULL argument");
    if (N <= 0 || K <= 0) return fail(GDN_ERR_SHAPE, "N=%d K=%d", N, K);
    HIP_OK(gdn::launch_quantize_e4m3(w, N, K, (u8*)q, scale, 0, as_stream(stream)));
    return GDN_OK;
}

int gdn_quantize_mxfp4(const void* w, int N, int K, void* q, void* scale, void* stream) {
    if (!w || !q || !scale) return fail(GDN_ERR_INVALID_ARG, "gdn_quantize_mxfp4: NULL argument");
    if (N <= 0 || K <= 0) return fail(GDN_ERR_SHAPE, "N=%d K=%d", N, K);
    if (K % 32) return fail(GDN_ERR_UNSUPPORTED, "K=%d is not a multiple of 32", K);
    HIP_OK(gdn::launch_quantize_mxfp4(w, N, K, (u8*)q, (u8*)scale, 0, as_stream(stream)));
    return GDN_OK;
}

int gdn_quantize_mxint8(const void* w, int N, int K, void* q, void* scale, void* stream) {
    if (!w || !q || !scale) return fail(GDN_ERR_INVALID_ARG, "gdn_quantize_mxint8: NULL argument");
    if (N <= 0 || K <= 0) return fail(GDN_ERR_SHAPE, "N=%d K=%d", N, K);
    if (K % 32) return fail(GDN_ERR_UNSUPPORTED, "K=%d is not a multiple of 32", K);
    HIP_OK(gdn::launch_quantize_mxint8(w, N, K, (u8*)q, (u8*)scale, 0, as_stream(stream)));
    return GDN_OK;
}

}  // extern "C"

// ------------------------------------------------------------------------------------------------
// Layer stack: the reference's Qwen35_08B_GDNStackL1 (wormhole_n150/qwen3.5_0.8B/gdn_l1.py:207-341) --
// layers of one geometry run back to back, each with its own weights and state slots, the output of
// layer i the input of layer i + 1 -- optionally with the decoder RMSNorm between layers.  The layers
// share one launch workspace; activations ping-pong between two buffers of the stack.
// ------------------------------------------------------------------------------------------------
struct gdn_stack {
    std::vector<gdn_layer*> layers;
    int inter_norm = 0;
    float* norm_w = nullptr;  // [n_layers, H] decoder RMSNorm weights (y = x rstd (1 + w))
    u16* act[2] = {nullptr, nullptr};
    int H = 0, max_tokens = 0;
    int out_kind = gdn::OUT_BF16;  // element type of the output of calls that run the last layer
    float eps = 1e-6f;
    ~gdn_stack() {
        for (size_t i = layers.size(); i-- > 0;) delete layers[i];  // borrowers before the workspace owner
        if (norm_w) (void)hipFree(norm_w);
        for (u16* a : act)
            if (a) (void)hipFree(a);
    }
};

namespace {

// Element type of `out` of a call over layers [first, first + count): the stack's output type when the call
// runs the last layer, else bf16 (the activations between layers, and the next call's input).
int stack_out_kind(const gdn_stack* S, int first, int count) {
    return first + count == (int)S->layers.size() ? S->out_kind : gdn::OUT_BF16;
}

// Layers [first, first + count) on rows made of `groups`; norms after every layer but the stack's last.
int stack_run(gdn_stack* S, const u16* x, int M, const Group* groups, int ng, int first, int count, void* out,
              hipStream_t st) {
    const u16* in = x;
    for (int i = first; i < first + count; ++i) {
        const bool last = i + 1 == first + count;
        u16* dst = last ? (u16*)out : S->act[(i - first) & 1];
        int rc = run_rows(S->layers[i], in, M, groups, ng, dst, last ? stack_out_kind(S, first, count) : gdn::OUT_BF16,
                          st);
        if (rc) return rc;
        if (S->inter_norm && i + 1 < (int)S->layers.size())
            HIP_OK(gdn::launch_rmsnorm_rows(dst, M, S->H, S->norm_w + (size_t)i * S->H, S->eps, dst, st));
        in = dst;
    }
    return GDN_OK;
}

}  // namespace

extern "C" {

int gdn_stack_create(const gdn_dims* dims, const gdn_weights* weights, int n_layers, int inter_norm,
                     const float* const* norm_weights, int max_slots, int max_tokens, gdn_stack** out) {
    return gdn_stack_create_ex(dims, weights, n_layers, inter_norm, norm_weights, max_slots, max_tokens,
                               GDN_WEIGHTS_BF16, out);
}

int gdn_stack_create_ex(const gdn_dims* dims, const gdn_weights* weights, int n_layers, int inter_norm,
                        const float* const* norm_weights, int max_slots, int max_tokens, int weight_format,
                        gdn_stack** out) {
    if (!out) return fail(GDN_ERR_INVALID_ARG, "out is NULL");
    *out = nullptr;
    if (!weights || n_layers <= 0) return fail(GDN_ERR_INVALID_ARG, "gdn_stack_create: %d layers", n_layers);
    int rc0 = check_dims(dims);
    if (rc0) return rc0;
    if (inter_norm && dims->hidden > 8192)
        return fail(GDN_ERR_UNSUPPORTED, "inter-layer RMSNorm over hidden %d (at most 8192)", dims->hidden);
    gdn_stack* S = new gdn_stack();
    for (int i = 0; i < n_layers; ++i) {
        gdn_layer* L = nullptr;
        int rc = create_layer(dims, &weights[i], max_slots, max_tokens, weight_format, i ? S->layers[0] : nullptr,
                              &L);
        if (rc) {
            delete S;
            return rc;
        }
        S->layers.push_back(L);
    }
    S->H = dims->hidden, S->max_tokens = max_tokens, S->inter_norm = inter_norm ? 1 : 0;
    S->eps = dims->rms_norm_eps;
    const size_t bytes = (size_t)max_tokens * S->H * sizeof(u16);
    hipError_t e = hipMalloc(&S->act[0], bytes);
    if (e == hipSuccess) e = hipMalloc(&S->act[1], bytes);
    if (e == hipSuccess) e = hipMalloc(&S->norm_w, (size_t)n_layers * S->H * sizeof(float));
    if (e == hipSuccess) e = hipMemset(S->norm_w, 0, (size_t)n_layers * S->H * sizeof(float));
    for (int i = 0; e == hipSuccess && norm_weights && i < n_layers; ++i)
        if (norm_weights[i])
            e = hipMemcpy(S->norm_w + (size_t)i * S->H, norm_weights[i], S->H * sizeof(float), hipMemcpyDefault);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        delete S;
        return fail(e == hipErrorOutOfMemory ? GDN_ERR_OUT_OF_MEMORY : GDN_ERR_HIP, "gdn_stack_create: %s",
                    hipGetErrorString(e));
    }
    *out = S;
    return GDN_OK;
}

int gdn_stack_destroy(gdn_stack* S) {
    if (!S) return GDN_OK;
    (void)hipDeviceSynchronize();
    delete S;
    return GDN_OK;
}

int gdn_stack_layer(gdn_stack* S, int i, gdn_layer** out) {
    if (!S || !out) return fail(GDN_ERR_INVALID_ARG, "gdn_stack_layer: NULL argument");
    if (i < 0 || i >= (int)S->layers.size()) return fail(GDN_ERR_INVALID_ARG, "layer %d of %zu", i, S->layers.size());
    *out = S->layers[i];
    return GDN_OK;
}

int gdn_stack_forward(gdn_stack* S, const void* x, int B, int T, const int* slot_ids, int first, int count,
                      void* out, void* stream) {
    if (!S || !x || !out) return fail(GDN_ERR_INVALID_ARG, "gdn_stack_forward: NULL argument");
    const int n = (int)S->layers.size();
    if (first < 0 || count <= 0 || first + count > n) return fail(GDN_ERR_INVALID_ARG, "layers [%d, %d) of %d", first, first + count, n);
    if (B <= 0 || T <= 0) return fail(GDN_ERR_SHAPE, "gdn_stack_forward: B=%d T=%d must be > 0", B, T);
    if (B > S->max_tokens) return fail(GDN_ERR_SHAPE, "B=%d exceeds max_tokens=%d", B, S->max_tokens);
    if (!slot_ids && B > S->layers[0]->max_slots) return fail(GDN_ERR_SLOT, "B=%d exceeds max_slots", B);
    const int* slots = slot_ids ? slot_ids : S->layers[0]->iota;
    const hipStream_t st = as_stream(stream);
    const u16* xin = (const u16*)x;
    char* xout = (char*)out;
    const int okind = stack_out_kind(S, first, count);
    const int tc_max = S->max_tokens / B;
    if (T <= tc_max) {
        const Group g{0, B, T, slots};
        return stack_run(S, xin, B * T, &g, 1, first, count, xout, st);
    }
    // Longer launches run token blocks of at most max_tokens rows through all the layers in turn: every layer
    // is causal and carries its states, so block by block equals the whole launch (9B/gdn_layer.py:282-292
    // splits one layer the same way).  Rows of several sequences are gathered into the workspace of layer 0
    // (not used by the layers' own launches) and scattered back.
    gdn_layer* L0 = S->layers[0];
    const size_t rb = (size_t)S->H * sizeof(u16), ob = (size_t)S->H * out_elem_bytes(okind);
    void* stage = split_out_stage(L0, okind);  // the layers share L0's workspaces
    if (B > 1 && !stage)
        return fail(GDN_ERR_UNSUPPORTED, "fp32 output of a split launch of %d sequences needs proj width %d >= "
                    "hidden %d", B, L0->NP, S->H);
    for (int t0 = 0; t0 < T; t0 += tc_max) {
        const int tc = T - t0 < tc_max ? T - t0 : tc_max;
        const Group g{0, B, tc, slots};
        if (B == 1) {
            int rc = stack_run(S, xin + (size_t)t0 * S->H, tc, &g, 1, first, count, xout + (size_t)t0 * ob, st);
            if (rc) return rc;
            continue;
        }
        HIP_OK(hipMemcpy2DAsync(L0->x_ws, tc * rb, xin + (size_t)t0 * S->H, (size_t)T * rb, tc * rb, B,
                                hipMemcpyDeviceToDevice, st));
        int rc = stack_run(S, L0->x_ws, B * tc, &g, 1, first, count, stage, st);
        if (rc) return rc;
        HIP_OK(hipMemcpy2DAsync(xout + (size_t)t0 * ob, (size_t)T * ob, stage, tc * ob, tc * ob, B,
                                hipMemcpyDeviceToDevice, st));
    }
    return GDN_OK;
}

int gdn_stack_forward_varlen(gdn_stack* S, const void* x, int n_seqs, const int* cu_seqlens, const int* slot_ids,
                             int first, int count, void* out, void* stream) {
    if (!S || !x || !out) return fail(GDN_ERR_INVALID_ARG, "gdn_stack_forward_varlen: NULL argument");
    const int n = (int)S->layers.size();
    if (first < 0 || count <= 0 || first + count > n) return fail(GDN_ERR_INVALID_ARG, "layers [%d, %d) of %d", first, first + count, n);
    std::vector<Group> groups;
    int rc = varlen_groups(S->layers[0], n_seqs, cu_seqlens, slot_ids, &groups);
    if (rc) return rc;
    return stack_run(S, (const u16*)x, cu_seqlens[n_seqs], groups.data(), (int)groups.size(), first, count, out,
                     as_stream(stream));
}

int gdn_stack_set_output_dtype(gdn_stack* S, int out_dtype) {
    if (!S) return fail(GDN_ERR_INVALID_ARG, "stack is NULL");
    if (out_dtype != GDN_OUT_BF16 && out_dtype != GDN_OUT_FP32)
        return fail(GDN_ERR_INVALID_ARG, "output dtype %d (GDN_OUT_BF16 = 0 or GDN_OUT_FP32 = 1)", out_dtype);
    S->out_kind = out_dtype == GDN_OUT_FP32 ? gdn::OUT_F32 : gdn::OUT_BF16;
    return GDN_OK;
}

}  // extern "C"

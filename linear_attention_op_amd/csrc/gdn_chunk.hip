// Chunked (64-token) gated delta rule for prefills: the WY / UT form of the recurrence on bf16 MFMA with
// the state carried in fp32.  Restates the chunk algorithm of HF torch_chunk_gated_delta_rule
// (transformers qwen3_5 modeling_qwen3_5.py:248-328, the layer truth the reference tests against,
// wormhole_n150/qwen3.5_9B/test_gdn_layer.py:42-73); it equals the token-by-token rule of
// wormhole_n150/qwen3.5_9B/reference.py:28-34 up to rounding.
//
// Per (sequence, v-head) and chunk of C = 64 tokens, with G = in-chunk cumulative log decay,
// Gam_ij = exp(G_i - G_j) (i >= j), normalised q, k, and the chunk's initial state S:
//     L    = strict_tril(beta k k^T (.) Gam)          T = (I + L)^-1            (fp32 forward substitution)
//     U    = T (beta V)                               W = T (beta K (.) e^G)
//     Aqk  = tril(q k^T (.) Gam)                      Q' = Q (.) e^G - Aqk W
//     O    = Q' S + Aqk U                             (= Q e^G S + Aqk (U - W S))
//     Vn   = U - W S
//     S   <- e^{G_last} S + (K (.) e^{G_last - G})^T Vn
//
// Two kernels:
//  * chunk_prep_kernel: every (sequence, v-head, chunk) in parallel.  Everything that does not depend on
//    S: G, L, T, U, W, Q', the decay-scaled transposed keys and the intra-chunk output Aqk U (into the
//    workspace, laid out as U).
//  * chunk_state_kernel: the sequential pass over chunks.  A workgroup owns 16 value columns of one
//    (sequence, v-head) state; its eight waves own 16 state rows each, held in MFMA accumulators for the
//    whole launch (state read once, written once).  Per chunk: the state goes through LDS as a bf16 hi|lo
//    MFMA operand; four waves form W S and Vn for one 16-token tile each, four form Q' S and O for one tile
//    each; then every wave updates its rows from Vn.  The operands of the next two chunks are in flight while
//    the current one is computed; each step issues the loads of the chunk two ahead in four parts spread
//    over its own work.  Workgroup ids put the 8 column blocks of a head on one XCD so that they share that
//    XCD's L2 copy of W, Q' and the keys.
//
// Precision: every product that feeds the state goes through split bf16 (hi + lo, three MFMAs, ~2^-17
// relative), so the chunked state matches the fp32 sequential rule to ~1e-5.  So does Q' S in the
// recurrence-only op (fp32 output); in the layer, whose output is bf16 after the gated norm, Q' is bf16
// alone (two MFMAs, S still split): output error 2.3-2.5e-3 against the fp64 oracle, as with split Q'.
#include <cmath>
#include <type_traits>

#include "gdn_common.h"

namespace gdn {

namespace {

constexpr int CK = 64;  // chunk length

__device__ __forceinline__ void load8(const float* p, float* v) {
    const float4 a = *reinterpret_cast<const float4*>(p);
    const float4 b = *reinterpret_cast<const float4*>(p + 4);
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
}

// The state pass's operands, written by the prep pass split into bf16 hi + lo (x = hi + lo) and in the
// exact per-lane order of the state pass's MFMA operands, so that the state pass loads each lane's
// fragment with one 16-byte access and converts nothing (lane = 16 grp + m):
struct ChunkWs {
    u16* Wf;    // [B, Hv, NC][4 rt][8 n][64 lane][8]: W[16 rt + m][16 n + 4 grp + j], hi j < 4, then lo
    u16* Qf;    // the same for Q'; in the layer (Q' in bf16 alone) [B, Hv, NC][4 rt][4 s][64 lane][8]:
                //   Q'[16 rt + m][32 s + 16 (j / 4) + 4 grp + j % 4] (hi)
    u16* Kf;    // [B, Hv, NC][8 w][2 s][2 plane][64 lane][8]: Kt[16 w + m][32 s + 8 grp + j], plane 0 hi, 1 lo
    float* U;   // [B, Hv, NC][4 mi][DV / 16 n][64 lane][4]: U[16 mi + 4 grp + i][16 n + m] (the prep pass's
                //   MFMA C order: one 16-byte store per lane; the state pass reads 8 contiguous bytes)
    float* O;   // the intra-chunk output M2 (beta V), laid out as U (in the output's own layout each lane's
                //   four rows would be four 4-byte stores, twice the prep pass's store instructions)
    float* G;   // [B, Hv, NC, CK]       G (in-chunk cumulative log decay)
    int NC;     // chunks per sequence
};

__device__ __forceinline__ uint32_t bf16_bits(float x) {
    return (uint32_t)__builtin_bit_cast(u16, (__bf16)x);
}

// ------------------------------------------------------------------------------------------------
// chunk_prep_kernel: grid (Hv, NC, B), 512 threads (8 waves, two per SIMD).
//
// Phases (wave w of 8; mi = w % 4 is a 16-token row tile, hf = w / 4 a half of the column tiles):
//   0. the chunk's inputs: thread (prow, pc4) owns tokens 4 prow .. 4 prow + 3, channels pc4 .. pc4 + 3 of
//      q, k, v (coalesced float4; in the layer computed by the fused front end), g, beta.
//   1. per-token normalisers (32-lane reductions), normalised keys -> sK (and kept in registers),
//      queries -> sQ (aliases the L / Aqk tiles, which are not written yet); G = cumsum(g).
//   2. k k^T and q k^T (wave w: row tile mi, column tiles 2 hf, 2 hf + 1 at or below it) -> L into sL,
//      Aqk into sA; the decay-scaled keys transposed through the key region into the state pass's key
//      fragments.
//   3. T = (I + L)^-1, blocked: the four 16 x 16 diagonal blocks by forward substitution (one wave
//      each), then T_ij = -T_ii sum_{k=j}^{i-1} L_ik T_kj by distance i - j = 1, 2, 3 -> sT.
//   4. M2 = Aqk T in place over Aqk.
//   5. T and M2 into registers; X = beta K e^G and beta V, from the keys and values still in registers,
//      transposed and split into the two regions; [T; M2] x X: W and Q' = Q e^G - Aqk W (wave w: row
//      tile mi, column tiles 4 hf .. 4 hf + 3).
//   6. [T; M2] x (beta V): U and the intra-chunk output.
// ------------------------------------------------------------------------------------------------
template <int DK, int DV, bool FUSED>
__global__ __launch_bounds__(512, 4) void chunk_prep_kernel(DeltaArgs a, ChunkWs ws, FrontArgs f) {
    static_assert(DK == 128 && DV == 128, "chunked path is specialised for 128-wide heads");
    constexpr int NT = 512;      // threads
    constexpr int LDK = DK + 4;  // row stride (floats) of the 64 x 128 tiles
    constexpr int LDT = CK + 4;  // row stride of the 64 x 64 tiles
    constexpr int LDX = 17;      // row stride of the 16 x 16 scratch blocks
    // Two regions, 68 KB with the scalars, so that two workgroups share a CU:
    //   sK:  keys (phases 1-2), transposed decay-scaled keys (2), T and the phase-3 scratch (3-5), X^T split (5)
    //   sLA: queries (1-2), then L | Aqk (M2) (2-5), then (beta V)^T split (5-6)
    __shared__ __attribute__((aligned(16))) float sK[CK * LDK];
    __shared__ __attribute__((aligned(16))) float sLA[2 * CK * LDT];
    __shared__ float sG[CK], sEG[CK], sDec[CK], sBeta[CK];
    static_assert(CK * LDT + 4 * 16 * LDX <= CK * LDK && CK * LDK <= 2 * CK * LDT && DK * CK <= CK * LDK,
                  "region sizes");
    float* sQ = sLA;                 // [CK][LDK] fits in the 2 * CK * LDT floats of sLA
    float* sL = sLA;                 // [CK][LDT]
    float* sA = sLA + CK * LDT;      // [CK][LDT]
    float* sT = sK;                  // [CK][LDT]
    float* sX = sK + CK * LDT;       // [4 waves][16 * LDX]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int mi = wave & 3, hf = wave >> 2;
    // heads fastest: the v-heads that share a k-head run back to back (on neighbouring XCDs), so the second
    // finds the k-head's rows in the memory-side cache
    const int h = blockIdx.x, c = blockIdx.y, b = blockIdx.z;
    const int T = a.T, Hk = a.Hk, Hv = a.Hv, kh = h / (Hv / Hk);
    const int t0 = c * CK, len = min(CK, T - t0);
    const size_t row0 = (size_t)b * T + t0;
    const int m = lane & 15, grp = lane >> 4;
    const size_t hc = ((size_t)b * Hv + h) * ws.NC + c;
    if (a.slot_ids && (unsigned)a.slot_ids[b] >= (unsigned)a.max_slots) return;

    // ---- 0. inputs: thread (prow, pc4) owns tokens 4 prow + j (j < 4), channels pc4 .. pc4 + 3 of q, k, v
    const int prow = tid >> 5, pc4 = (tid & 31) * 4;
    // v if ok, else zeros: per-component selects after an unconditional load from a valid address (a select
    // between a loaded and a constant vector would be turned into a load from a private copy of the constant)
    auto keep_if = [](bool ok, float4 v) {
        return make_float4(ok ? v.x : 0.f, ok ? v.y : 0.f, ok ? v.z : 0.f, ok ? v.w : 0.f);
    };
    float4 kr[4], vr[4];
    float gv = 0.f, bv = 0.f;
    // l2norm over the 32 lanes of a half-wave (one token's row), times `mult`, and the row into LDS
    auto l2store = [&](float4* x, float mult, float* dst) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float ss = x[j].x * x[j].x + x[j].y * x[j].y + x[j].z * x[j].z + x[j].w * x[j].w;
#pragma unroll
            for (int off = 1; off < 32; off <<= 1) ss += __shfl_xor(ss, off, 64);
            const float r = (a.normalize ? rsqrtf(ss + 1e-6f) : 1.f) * mult;
            x[j].x *= r, x[j].y *= r, x[j].z *= r, x[j].w *= r;
            *reinterpret_cast<float4*>(&dst[(4 * prow + j) * LDK + pc4]) = x[j];
        }
    };
    // The fused front end (FUSED), from the projection rows: causal conv (4 taps over the inputs at t - 3 .. t,
    // the slot's history before t = 0) + SiLU, as conv_front_kernel (layer_compute.cpp C1, 74-103).  The window
    // of the thread's 4 tokens is 7 input rows, loaded one tensor at a time (register budget).
    const int R = Hv / Hk;
    const int Kd = f.nk * DK, Vd = f.nv * DV, CD = 2 * Kd + Vd, CH = conv_group_width(DK, DV, R);
    const float* hg = nullptr;  // the k-head group's history ring (q and k of kh, v of this head at 2 DK + (h % R) DV)
    int pos = 0;
    if constexpr (FUSED) {
        const int slot = f.slot_ids ? f.slot_ids[b] : b;
        hg = f.conv_state + ((size_t)slot * f.nk + kh) * CONV_RING * CH;
        pos = f.conv_pos[(size_t)slot * f.nv + h];
    }
    const int colq = kh * DK + pc4, colk = Kd + kh * DK + pc4, colv = 2 * Kd + h * DV + pc4;
    const int locv = 2 * DK + (h % R) * DV + pc4;
    auto in_row = [&](int tk, int col, int local) -> float4 {
        const int tkc = min(tk, len - 1);  // rows past the end read a valid row, zeroed below
        const int t = t0 + tkc;
        const float* p = t >= 0 ? f.P + (size_t)((long long)row0 + tkc) * f.NP + col
                                : hg + ring_index(pos, 3 + t) * CH + local;
        return keep_if(tk < len, *reinterpret_cast<const float4*>(p));
    };
    auto window = [&](int col, int local, float4* x) {
#pragma unroll
        for (int r = 0; r < 7; ++r) x[r] = in_row(4 * prow - 3 + r, col, local);
    };
    auto convolve = [&](int col, const float4* x, float4* out) {
        float4 w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = f.conv_w[col + i];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float4 x0 = x[j], x1 = x[j + 1], x2 = x[j + 2], x3 = x[j + 3];
            float4 o;
            o.x = siluf_(w[0].x * x0.x + w[0].y * x1.x + w[0].z * x2.x + w[0].w * x3.x);
            o.y = siluf_(w[1].x * x0.y + w[1].y * x1.y + w[1].z * x2.y + w[1].w * x3.y);
            o.z = siluf_(w[2].x * x0.z + w[2].y * x1.z + w[2].z * x2.z + w[2].w * x3.z);
            o.w = siluf_(w[3].x * x0.w + w[3].y * x1.w + w[3].z * x2.w + w[3].w * x3.w);
            out[j] = keep_if(4 * prow + j < len, o);
        }
    };
    if constexpr (FUSED) {
        if (wave == 0 && lane < len) {
            const float* Pr = f.P + (row0 + lane) * f.NP + CD + Vd;
            gv = f.neg_A[h] * softplusf_(Pr[h] + f.dt_bias[h]);
            bv = sigmoidf_(Pr[f.nv + h]);
        }
        // the queries normalised and stored before the keys' window is loaded
        {
            float4 x[7], qr[4];
            window(colq, pc4, x);
            convolve(colq, x, qr);
            l2store(qr, a.scale, sQ);
        }
        {
            float4 x[7];
            window(colk, DK + pc4, x);
            convolve(colk, x, kr);
        }
        l2store(kr, 1.f, sK);
        {
            float4 x[7];
            window(colv, locv, x);
            convolve(colv, x, vr);
        }
    } else {
        float4 qr[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int tok = 4 * prow + j;
            const bool ok = tok < len;
            const size_t row = row0 + (ok ? tok : 0);
            const size_t qk = (row * Hk + kh) * DK + pc4;
            kr[j] = keep_if(ok, *reinterpret_cast<const float4*>(a.k + qk));
            qr[j] = keep_if(ok, *reinterpret_cast<const float4*>(a.q + qk));
            vr[j] = keep_if(ok, *reinterpret_cast<const float4*>(a.v + (row * Hv + h) * DV + pc4));
        }
        if (wave == 0 && lane < len) gv = a.g[(row0 + lane) * Hv + h], bv = a.beta[(row0 + lane) * Hv + h];
        l2store(qr, a.scale, sQ);
        l2store(kr, 1.f, sK);
    }
    // (the normalised keys stay in registers)

    // ---- 1. G ---------------------------------------------------------------------------------------------
    if (wave == 0) {
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const float y = __shfl_up(gv, off, 64);
            if (lane >= off) gv += y;
        }
        sG[lane] = gv;
        sEG[lane] = __expf(gv);
        sDec[lane] = __expf(__shfl(gv, CK - 1, 64) - gv);
        sBeta[lane] = bv;
    }
    __syncthreads();

    // ---- 2. k k^T and q k^T: wave w owns row tile mi, column tiles 2 hf, 2 hf + 1 -----------------------
    float4 qe[4];
    {
        f32x4 akk[2], aqk[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) akk[q] = aqk[q] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (2 * hf <= mi) {
#pragma unroll
            for (int s = 0; s < DK / 32; ++s) {
                const int k0 = 32 * s + 8 * grp;
                float ka[8], qa[8];
                load8(&sK[(16 * mi + m) * LDK + k0], ka);
                load8(&sQ[(16 * mi + m) * LDK + k0], qa);
                const Split8 A1 = split8(ka), A2 = split8(qa);
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    const int ni = 2 * hf + q;
                    if (ni > mi) continue;
                    float kb[8];
                    load8(&sK[(16 * ni + m) * LDK + k0], kb);
                    const Split8 Bk = split8(kb);
                    akk[q] = mfma3(A1, Bk, akk[q]);
                    aqk[q] = mfma3(A2, Bk, aqk[q]);
                }
            }
        }
        // the queries this wave needs later for Q' (token 16 mi + m, columns 16 n + 4 grp + i for its column
        // tiles n = 4 hf .. 4 hf + 3: the C layout of the transposed product in phase 5), before sQ is
        // overwritten
#pragma unroll
        for (int n = 0; n < 4; ++n)
            qe[n] = *reinterpret_cast<const float4*>(&sQ[(16 * mi + m) * LDK + 16 * (4 * hf + n) + 4 * grp]);
        __syncthreads();  // every wave is done with sK and sQ before they are overwritten
        // Kt[r][tok] = k[tok][r] e^{G_last - G_tok} (the state pass's keys) transposed into the key region, fp32
        // with 16-byte chunks xor-swizzled: element (r, tok) at r * CK + ((tok / 4) ^ ((r / 4) % 16)) * 4 +
        // tok % 4 (thread (prow, pc4) holds tokens 4 prow + j of channels pc4 + cc: one chunk per channel)
        {
            float dec[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) dec[j] = sDec[4 * prow + j];
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) {
                const int r = pc4 + cc;
                float4 v;
                v.x = (cc == 0 ? kr[0].x : (cc == 1 ? kr[0].y : (cc == 2 ? kr[0].z : kr[0].w))) * dec[0];
                v.y = (cc == 0 ? kr[1].x : (cc == 1 ? kr[1].y : (cc == 2 ? kr[1].z : kr[1].w))) * dec[1];
                v.z = (cc == 0 ? kr[2].x : (cc == 1 ? kr[2].y : (cc == 2 ? kr[2].z : kr[2].w))) * dec[2];
                v.w = (cc == 0 ? kr[3].x : (cc == 1 ? kr[3].y : (cc == 2 ? kr[3].z : kr[3].w))) * dec[3];
                *reinterpret_cast<float4*>(&sK[r * CK + ((prow ^ ((r >> 2) & 15)) << 2)]) = v;
            }
        }
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int ni = 2 * hf + q;
                const int r = 16 * mi + 4 * grp + i, cc = 16 * ni + m;
                float L = 0.f, A = 0.f;
                if (ni <= mi && cc <= r) {
                    const float dec = __expf(sG[r] - sG[cc]);
                    A = aqk[q][i] * dec;
                    if (cc < r) L = sBeta[r] * akk[q][i] * dec;
                }
                sL[r * LDT + cc] = L;
                sA[r * LDT + cc] = A;
            }
    }
    __syncthreads();

    // The state pass's key fragments from the transposed keys: thread t writes units t and t + 512 of the
    // chunk's Kf block (unit u: row r = 16 (u / 128) + u % 16, 8-token group 4 ((u / 64) % 2) + (u / 16) % 4;
    // 16 bytes into each plane of its 64-unit block), so that a wave writes two 1 KB runs.
    {
        u16* Kf = ws.Kf + hc * DK * CK * 2;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int u = tid + NT * e;
            const int r = 16 * (u >> 7) + (u & 15), tg = 4 * ((u >> 6) & 1) + ((u >> 4) & 3), sw = (r >> 2) & 15;
            float x[8];
            const float4 a0 = *reinterpret_cast<const float4*>(&sK[r * CK + (((2 * tg) ^ sw) << 2)]);
            const float4 a1 = *reinterpret_cast<const float4*>(&sK[r * CK + (((2 * tg + 1) ^ sw) << 2)]);
            x[0] = a0.x, x[1] = a0.y, x[2] = a0.z, x[3] = a0.w, x[4] = a1.x, x[5] = a1.y, x[6] = a1.z, x[7] = a1.w;
            u16x8 hi, lo;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const __bf16 xh = (__bf16)x[j];
                hi[j] = __builtin_bit_cast(u16, xh);
                lo[j] = (u16)bf16_bits(x[j] - (float)xh);
            }
            *reinterpret_cast<u16x8*>(Kf + (size_t)(u >> 6) * 1024 + (u & 63) * 8) = hi;
            *reinterpret_cast<u16x8*>(Kf + (size_t)(u >> 6) * 1024 + 512 + (u & 63) * 8) = lo;
        }
    }

    // ---- 3. T = (I + L)^-1 ---------------------------------------------------------------------------
    // 3a. diagonal block w (waves 0-3): lane c < 16 owns column c, rows by forward substitution (into
    //     registers; written after every wave has read the transposed keys that T overwrites)
    float t[16];
    if (wave < 4 && lane < 16) {
        const int o = 16 * wave;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            float acc = (r == lane) ? 1.f : 0.f;
#pragma unroll
            for (int k = 0; k < r; ++k) acc -= sL[(o + r) * LDT + o + k] * t[k];
            t[r] = acc;
        }
    }
    __syncthreads();
    if (wave < 4 && lane < 16) {
#pragma unroll
        for (int r = 0; r < 16; ++r) sT[(16 * wave + r) * LDT + 16 * wave + lane] = t[r];
    }
    // upper blocks of T are zero
    for (int e = tid; e < CK * CK; e += NT) {
        const int r = e / CK, cc = e % CK;
        if ((cc >> 4) > (r >> 4)) sT[r * LDT + cc] = 0.f;
    }
    __syncthreads();
    // 3b. T_ij = -T_ii X, X = sum_{k=j}^{i-1} L_ik T_kj (wave j, i = j + dist), on 16x16x4 fp32 MFMAs (fp32
    //     products like the substitution above): A lane (m, grp) = L[16 i + m][16 k + 4 s + grp], B lane (m, grp)
    //     = T[16 k + 4 s + grp][16 j + m].  X leaves in the C layout (rows 4 grp + r of column m) and passes
    //     through the wave's scratch block to become the B operand of T_ii X.
#pragma unroll
    for (int dist = 1; dist < 4; ++dist) {
        const int j = wave, i = wave + dist;
        if (i < 4) {
            f32x4 x = {0.f, 0.f, 0.f, 0.f};
            for (int k = j; k < i; ++k)
#pragma unroll
                for (int s = 0; s < 4; ++s)
                    x = __builtin_amdgcn_mfma_f32_16x16x4f32(sL[(16 * i + m) * LDT + 16 * k + 4 * s + grp],
                                                            sT[(16 * k + 4 * s + grp) * LDT + 16 * j + m], x, 0, 0, 0);
            float* xs = sX + wave * 16 * LDX;
#pragma unroll
            for (int r = 0; r < 4; ++r) xs[(4 * grp + r) * LDX + m] = x[r];
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            f32x4 y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < 4; ++s)
                y = __builtin_amdgcn_mfma_f32_16x16x4f32(sT[(16 * i + m) * LDT + 16 * i + 4 * s + grp],
                                                        xs[(4 * s + grp) * LDX + m], y, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r) sT[(16 * i + 4 * grp + r) * LDT + 16 * j + m] = -y[r];
        }
        __syncthreads();
    }

    // ---- 4. M2 = Aqk T, in place over Aqk: wave w makes tiles (mi, 2 hf), (mi, 2 hf + 1) at or below the
    //      diagonal (tiles above it stay zero); both waves of a row tile read all of it first --------------
    {
        f32x4 acc[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) acc[q] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (2 * hf <= mi) {
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                if (32 * s > 16 * mi + 15) continue;  // Aqk row tile mi is zero past column 16 mi + 15
                const int k0 = 32 * s + 8 * grp;
                float av[8];
                load8(&sA[(16 * mi + m) * LDT + k0], av);
                const Split8 A = split8(av);
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    const int ni = 2 * hf + q;
                    if (ni > mi || 32 * s + 31 < 16 * ni) continue;  // T column tile ni is zero above row 16 ni
                    float tb[8];
#pragma unroll
                    for (int jj = 0; jj < 8; ++jj) tb[jj] = sT[(k0 + jj) * LDT + 16 * ni + m];
                    acc[q] = mfma3(A, split8(tb), acc[q]);
                }
            }
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int ni = 2 * hf + q;
            if (ni > mi) continue;
#pragma unroll
            for (int i = 0; i < 4; ++i) sA[(16 * mi + 4 * grp + i) * LDT + 16 * ni + m] = acc[q][i];
        }
    }
    __syncthreads();

    // ---- 5, 6. [T; M2] x (beta K e^G | beta V) -----------------------------------------------------------
    // X = beta K e^G and beta V, transposed and split into bf16 hi | lo planes, from the keys and values in
    // registers (thread (prow, pc4): tokens 4 prow + j of channels pc4 + cc, half `prow % 2` of the 8-token
    // group prow / 2).  Element (r, tok) at r * CK + ((tok / 8) ^ ((r / 4) % 8)) * 8 + tok % 8.  A store
    // instruction writes rows 4 l + cc (l < 32, one cc): keyed on r / 4 the xor spreads them over eight 16-byte
    // slots (4-way bank conflicts; keyed on r % 8, two slots and 16-way), and the 16-byte fragment reads below
    // stay at two lanes per bank group.
    // Order, for the register budget: X^T goes where L and the phase-3 scratch were (its hi plane after T in
    // the key region, its lo plane over L) while T and M2 are still in LDS, so the keys leave the registers
    // before T and M2 enter them; W and Q' follow (the queries leave); then (beta V)^T goes over T and M2.
    u16* XTh = reinterpret_cast<u16*>(sK + CK * LDT);
    u16* XTl = reinterpret_cast<u16*>(sL);
    u16* VTh = reinterpret_cast<u16*>(sT);
    u16* VTl = reinterpret_cast<u16*>(sA);
    static_assert(DK * CK <= 2 * (CK * LDK - CK * LDT) && DV * CK <= 2 * CK * LDT, "X^T / V^T planes");
    auto put_t = [&](u16* hp, u16* lp, const float4* x, const float* sc) {
        const int tg = prow >> 1, half = (prow & 1) * 4;
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
            const int r = pc4 + cc;
            u16x4 h4, l4;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float v = (cc == 0 ? x[j].x : (cc == 1 ? x[j].y : (cc == 2 ? x[j].z : x[j].w))) * sc[j];
                const __bf16 vh = (__bf16)v;
                h4[j] = __builtin_bit_cast(u16, vh);
                l4[j] = (u16)bf16_bits(v - (float)vh);
            }
            const int o = r * CK + ((tg ^ ((r >> 2) & 7)) << 3) + half;
            *reinterpret_cast<u16x4*>(hp + o) = h4;
            *reinterpret_cast<u16x4*>(lp + o) = l4;
        }
    };
    {
        float sc[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) sc[j] = sBeta[4 * prow + j] * sEG[4 * prow + j];
        put_t(XTh, XTl, kr, sc);
    }
    const int nks = (16 * mi + 15 >= 32) ? 2 : 1;  // row tile mi of T and M2 is zero past column 16 mi + 15
    Split8 At[2], Am[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        if (s >= nks) continue;
        float tv[8], mv[8];
        load8(&sT[(16 * mi + m) * LDT + 32 * s + 8 * grp], tv);
        load8(&sA[(16 * mi + m) * LDT + 32 * s + 8 * grp], mv);
        At[s] = split8(tv);
        Am[s] = split8(mv);
    }
    __syncthreads();  // X^T is complete; T and M2 are in registers, so their regions are free
    // operand of token group (4 s + grp) for row r (16-byte reads, the xor layout above)
    auto tfrag = [&](const u16* hp, const u16* lp, int r, int s) {
        const int o = r * CK + (((4 * s + grp) ^ ((r >> 2) & 7)) << 3);
        return Split8{*reinterpret_cast<const bf16x8*>(hp + o), *reinterpret_cast<const bf16x8*>(lp + o)};
    };

    // 5. W and Q' as transposed products (X^T T^T and X^T M2^T: the operands of [T; M2] X swapped), whose
    //    C layout is the state pass's A-operand layout: lane (m, grp) holds W[16 mi + m][16 n + 4 grp + i]
    u16* Wf = ws.Wf + hc * CK * DK * 2;
    u16* Qf = ws.Qf + hc * CK * DK * 2;
    const float egm = sEG[16 * mi + m];
    const bool tok_ok = 16 * mi + m < len;
#pragma unroll
    for (int nn = 0; nn < 4; ++nn) {
        const int n = 4 * hf + nn;
        f32x4 accT = {0.f, 0.f, 0.f, 0.f}, accM = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            if (s >= nks) continue;
            const Split8 X = tfrag(XTh, XTl, 16 * n + m, s);
            accT = mfma3(X, At[s], accT);
            accM = mfma3(X, Am[s], accM);
        }
        const float qv[4] = {qe[nn].x, qe[nn].y, qe[nn].z, qe[nn].w};
        u16x8 fw, fq;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float wv = accT[i];
            const float qq = tok_ok ? qv[i] * egm - accM[i] : 0.f;
            const __bf16 wh = (__bf16)wv, qh = (__bf16)qq;
            fw[i] = __builtin_bit_cast(u16, wh);
            fw[4 + i] = (u16)bf16_bits(wv - (float)wh);
            fq[i] = __builtin_bit_cast(u16, qh);
            fq[4 + i] = (u16)bf16_bits(qq - (float)qh);
        }
        const size_t f8 = ((size_t)(mi * 8 + n) * 64 + lane) * 8;
        *reinterpret_cast<u16x8*>(Wf + f8) = fw;
        if constexpr (FUSED) {
            // the layer: Q' in bf16 alone (it only feeds the output).  Column tiles 2 s and 2 s + 1 fill the two
            // halves of one 16-byte fragment, k-slice s of the state pass's 16x16x32 operand
            const u16x4 qh4 = {fq[0], fq[1], fq[2], fq[3]};
            *reinterpret_cast<u16x4*>(Qf + ((size_t)(mi * 4 + (n >> 1)) * 64 + lane) * 8 + 4 * (n & 1)) = qh4;
        } else {
            *reinterpret_cast<u16x8*>(Qf + f8) = fq;
        }
    }
    {
        float bt[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) bt[j] = sBeta[4 * prow + j];
        put_t(VTh, VTl, vr, bt);
    }
    __syncthreads();  // (beta V)^T is complete
    // 6. U = T (beta V) (lane (m, grp): tokens 16 mi + 4 grp + i of column 16 n + m) and the intra-chunk
    //    output M2 (beta V), both in U's layout
    float* U = ws.U + hc * CK * DV;
    float* O = ws.O + hc * CK * DV;
#pragma unroll
    for (int nn = 0; nn < 4; ++nn) {
        const int n = 4 * hf + nn, col = 16 * n + m;
        f32x4 accT = {0.f, 0.f, 0.f, 0.f}, accM = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            if (s >= nks) continue;
            const Split8 V = tfrag(VTh, VTl, col, s);
            accT = mfma3(At[s], V, accT);
            accM = mfma3(Am[s], V, accM);
        }
        *reinterpret_cast<f32x4*>(U + ((size_t)(mi * (DV / 16) + n) * 64 + lane) * 4) = accT;
        *reinterpret_cast<f32x4*>(O + ((size_t)(mi * (DV / 16) + n) * 64 + lane) * 4) = accM;
    }
    if (tid < CK) ws.G[hc * CK + tid] = sG[tid];
}

// ------------------------------------------------------------------------------------------------
// chunk_state_kernel: grid (Hv * DV / 16, B), 512 threads.  blockIdx.x = cb * Hv + h.
//
// Wave w holds state rows 16 w .. 16 w + 15 of the workgroup's 16 columns in an MFMA accumulator for the
// whole launch.  Per chunk, with the chunk's initial state S in LDS as the B operand of a 16x16x32 MFMA:
//   phase 1: waves 0-3 form W S for token tile w (K = 128: four k-slices, split bf16, three MFMAs each)
//            and put Vn = U - W S into LDS; waves 4-7 form Q' S for token tile w - 4 and store
//            O = O_intra + Q' S.
//   phase 2: every wave updates its rows, S <- e^{G_last} S + (K e^{G_last - G})^T Vn, and puts them into LDS
//            for the next chunk.
// A barrier ends each phase.  Splitting phase 1 by token tile keeps each product whole in one accumulator,
// so LDS carries the state (8 KB written per chunk) and Vn (4 KB) but no partial sums.
// ------------------------------------------------------------------------------------------------

// One chunk's operands for one lane of a W wave (W_ROLE) or a Q' wave.  QSPLIT: Q' as bf16 hi and lo (the
// recurrence-only op, whose fp32 output is held to 1e-3), else hi alone (the layer, whose output is bf16
// after the gated norm; Q' does not enter the state).
template <bool QSPLIT, bool W_ROLE>
struct StateOps {
    static constexpr int NA = (W_ROLE || QSPLIT) ? 8 : 4;
    u16x8 a[NA];          // the token tile's W (or Q') fragments: [n] hi | lo, or (Q' hi alone) [s]
    u16x8 kh[2], kl[2];   // Kt [16 wave + m][32 s + 8 grp + j] (hi / lo)
    f32x4 uo;             // U (or the intra-chunk output) of the token tile, C layout
    float glast;          // G of the chunk's last token
};

template <int DK, int DV, bool QSPLIT>
__global__ __launch_bounds__(512) void chunk_state_kernel(DeltaArgs a, ChunkWs ws) {
    static_assert(DK == 128 && DV == 128, "chunked path is specialised for 128-wide heads");
    // The chunk's initial state as the B operand of W S and Q' S: k-slice s, plane (hi, lo), lane (m, grp),
    // slot j holds S[32 s + 16 (j / 4) + 4 grp + j % 4][n0 + m] (the k order of the W and Q' fragments), so
    // wave w's accumulator is slots 4 (w % 2) .. 4 (w % 2) + 3 of slice w / 2, one 8-byte store per plane.
    __shared__ __attribute__((aligned(16))) u16 sS[4][2][64][8];
    // Vn split into bf16 hi | lo, in the update's B-operand order: token t at [t / 32][(t / 8) % 4][col][t % 8]
    __shared__ __attribute__((aligned(16))) u16 vnf[2][4][16][16];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int Hv = a.Hv, T = a.T;
    const int h = blockIdx.x % Hv, cb = blockIdx.x / Hv, b = blockIdx.y;
    const int n0 = 16 * cb;
    const int slot = a.slot_ids ? a.slot_ids[b] : b;
    if ((unsigned)slot >= (unsigned)a.max_slots) return;
    const int m = lane & 15, grp = lane >> 4;
    const int NC = (T + CK - 1) / CK;
    const int rt = wave & 3;  // phase 1 token tile

    // this wave's 16 state rows 16 w + 4 grp + i (i < 4), column n0 + m: the C layout of the 16x16 MFMA, so
    // the update accumulates in place
    float* S = a.state + ((size_t)slot * Hv + h) * DK * DV;
    f32x4 st;
#pragma unroll
    for (int i = 0; i < 4; ++i) st[i] = S[(size_t)(16 * wave + 4 * grp + i) * DV + n0 + m];
    auto put_state = [&]() {
        u16x4 hi, lo;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const __bf16 x = (__bf16)st[i];
            hi[i] = __builtin_bit_cast(u16, x);
            lo[i] = (u16)bf16_bits(st[i] - (float)x);
        }
        *reinterpret_cast<u16x4*>(&sS[wave >> 1][0][lane][4 * (wave & 1)]) = hi;
        *reinterpret_cast<u16x4*>(&sS[wave >> 1][1][lane][4 * (wave & 1)]) = lo;
    };
    put_state();

    // The two roles run the same sequence of barriers with their own operands, each as straight-line code
    // (no role test between a load and its use).  The role is uniform over a wave (the wave index is a
    // scalar), and both loops pass the same two barriers per chunk for the same chunk count, so every wave
    // of the workgroup meets every barrier.
    auto run = [&](auto role) {
        constexpr bool WR = decltype(role)::value;
        using Ops = StateOps<QSPLIT, WR>;
        constexpr int NA = Ops::NA;
        const u16* abase = (WR ? ws.Wf : ws.Qf) + (size_t)rt * NA * 512 + lane * 8;
        const float* uobase = (WR ? ws.U : ws.O) + ((size_t)(rt * (DV / 16) + cb) * 64 + lane) * 4;
        float* obase = a.o + ((size_t)b * T * Hv + h) * DV + n0 + m;

        // One chunk's operands, loaded in four parts; a step issues the parts of the chunk two ahead at four
        // points of its own work, so the address units stream them while it computes.
        auto load_part = [&](int c, Ops& op, auto part) {
            constexpr int P = decltype(part)::value;
            const size_t hc = ((size_t)b * Hv + h) * ws.NC + c;
            if constexpr (P == 0 || P == 1) {
                const u16* src = abase + hc * CK * DK * 2;
#pragma unroll
                for (int i = P * NA / 2; i < (P + 1) * NA / 2; ++i)
                    op.a[i] = *reinterpret_cast<const u16x8*>(src + (size_t)i * 512);
            } else if constexpr (P == 2) {
                const size_t kf = hc * DK * CK * 2 + (size_t)wave * 2 * 1024 + lane * 8;
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    op.kh[s] = *reinterpret_cast<const u16x8*>(ws.Kf + kf + (size_t)s * 1024);
                    op.kl[s] = *reinterpret_cast<const u16x8*>(ws.Kf + kf + (size_t)s * 1024 + 512);
                }
            } else {
                op.uo = *reinterpret_cast<const f32x4*>(uobase + hc * CK * DV);
                op.glast = ws.G[hc * CK + CK - 1];
            }
        };
        using P0 = std::integral_constant<int, 0>;
        using P1 = std::integral_constant<int, 1>;
        using P2 = std::integral_constant<int, 2>;
        using P3 = std::integral_constant<int, 3>;
        auto load_ops = [&](int c, Ops& op) {
            load_part(c, op, P0{});
            load_part(c, op, P1{});
            load_part(c, op, P2{});
            load_part(c, op, P3{});
        };
        // part P of the loads into `nxt` (when LD), fenced so that the scheduler keeps it at this point
        auto issue = [&](int cn, Ops& nxt, auto ld, auto part) {
            if constexpr (decltype(ld)::value) {
                __builtin_amdgcn_sched_barrier(0);
                load_part(cn, nxt, part);
                __builtin_amdgcn_sched_barrier(0);
            }
        };

        // FULL: the chunk has CK tokens (no per-token bounds test)
        // LD: load chunk cn into nxt along the way
        auto step = [&](int c, const Ops& cur, auto full, int cn, Ops& nxt, auto ld) {
            constexpr bool FULL = decltype(full)::value;
            const int t0 = c * CK, len = FULL ? CK : min(CK, T - t0);
            issue(cn, nxt, ld, P0{});

            // phase 1: W S (Q' S) for token tile rt over the four k-slices of the state
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const Split8 Sb{__builtin_bit_cast(bf16x8, *reinterpret_cast<const u16x8*>(&sS[s][0][lane][0])),
                                __builtin_bit_cast(bf16x8, *reinterpret_cast<const u16x8*>(&sS[s][1][lane][0]))};
                if constexpr (NA == 8) {
                    // k-blocks 2 s and 2 s + 1 (four hi, four lo each) joined into the slice's hi and lo
                    const u16x8 x = cur.a[2 * s], y = cur.a[2 * s + 1];
                    const Split8 A{__builtin_bit_cast(bf16x8, __builtin_shufflevector(x, y, 0, 1, 2, 3, 8, 9, 10, 11)),
                                   __builtin_bit_cast(bf16x8, __builtin_shufflevector(x, y, 4, 5, 6, 7, 12, 13, 14, 15))};
                    acc = mfma3(A, Sb, acc);
                } else {
                    const bf16x8 qa = __builtin_bit_cast(bf16x8, cur.a[s]);
                    acc = mfma16(qa, Sb.h, mfma16(qa, Sb.l, acc));
                }
            }
            if constexpr (WR) {
                // Vn = U - W S for tokens 16 rt + 4 grp + i of column n0 + m
                u16x4 hi, lo;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float v = cur.uo[i] - acc[i];
                    const __bf16 x = (__bf16)v;
                    hi[i] = __builtin_bit_cast(u16, x);
                    lo[i] = (u16)bf16_bits(v - (float)x);
                }
                const int t = 16 * rt + 4 * grp;
                u16* vp = &vnf[t >> 5][(t >> 3) & 3][m][t & 7];
                *reinterpret_cast<u16x4*>(vp) = hi;
                *reinterpret_cast<u16x4*>(vp + 8) = lo;
            } else {
                // O = O_intra + Q' S for the same tokens
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int t = 16 * rt + 4 * grp + i;
                    if (FULL || t < len) obase[(size_t)(t0 + t) * Hv * DV] = cur.uo[i] + acc[i];
                }
            }
            issue(cn, nxt, ld, P1{});
            lds_barrier();

            // phase 2: S <- e^{G_last} S + (K e^{G_last - G})^T Vn
            issue(cn, nxt, ld, P2{});
            const float egl = __expf(cur.glast);
#pragma unroll
            for (int i = 0; i < 4; ++i) st[i] *= egl;
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                const u16x8 vh = *reinterpret_cast<const u16x8*>(&vnf[s][grp][m][0]);
                const u16x8 vl = *reinterpret_cast<const u16x8*>(&vnf[s][grp][m][8]);
                const Split8 kt{__builtin_bit_cast(bf16x8, cur.kh[s]), __builtin_bit_cast(bf16x8, cur.kl[s])};
                const Split8 vs{__builtin_bit_cast(bf16x8, vh), __builtin_bit_cast(bf16x8, vl)};
                st = mfma3(kt, vs, st);
            }
            put_state();
            issue(cn, nxt, ld, P3{});
            lds_barrier();
        };

        // Operands two chunks ahead: a 3-slot ring, unrolled so that every slot is a fixed set of registers.
        // The main loop runs over whole triples of full chunks with no conditional memory operation (loads
        // past the last chunk re-read the last chunk), so the only waits are for the oldest slot's loads;
        // the remaining (at most 3, the last possibly partial) chunks follow.
        using Full = std::integral_constant<bool, true>;
        using Part = std::integral_constant<bool, false>;
        using Yes = std::integral_constant<bool, true>;
        using No = std::integral_constant<bool, false>;
        const int NCF = T / CK;  // full chunks
        Ops A, B, C;
        load_ops(0, A);
        load_ops(min(1, NC - 1), B);
        lds_barrier();  // the initial state is in LDS
        int c = 0;
        for (; c + 3 <= NCF; c += 3) {
            step(c, A, Full{}, min(c + 2, NC - 1), C, Yes{});
            step(c + 1, B, Full{}, min(c + 3, NC - 1), A, Yes{});
            step(c + 2, C, Full{}, min(c + 4, NC - 1), B, Yes{});
        }
        if (c < NC) {
            step(c, A, Part{}, min(c + 2, NC - 1), C, Yes{});
            if (c + 1 < NC) {
                step(c + 1, B, Part{}, 0, A, No{});
                if (c + 2 < NC) step(c + 2, C, Part{}, 0, A, No{});
            }
        }
    };
    if (wave < 4) run(std::true_type{});
    else run(std::false_type{});

#pragma unroll
    for (int i = 0; i < 4; ++i) S[(size_t)(16 * wave + 4 * grp + i) * DV + n0 + m] = st[i];
}

}  // namespace

// Carve the workspace of a launch (128-wide heads).
static ChunkWs chunk_ws(const DeltaArgs& a, void* workspace) {
    constexpr int D = 128;
    ChunkWs ws;
    ws.NC = (a.T + CK - 1) / CK;
    const size_t n = (size_t)a.B * a.Hv * ws.NC;
    u16* p = static_cast<u16*>(workspace);
    ws.Wf = p, p += n * CK * D * 2;
    ws.Qf = p, p += n * CK * D * 2;
    ws.Kf = p, p += n * CK * D * 2;
    float* f = reinterpret_cast<float*>(p);
    ws.U = f, f += n * CK * D;
    ws.O = f, f += n * CK * D;
    ws.G = f;
    return ws;
}

size_t delta_chunked_workspace(int B, int T, int Hv, int dk, int dv) {
    const size_t NC = (size_t)(T + CK - 1) / CK;
    // W, Q', keys: bf16 hi + lo (4 bytes per value); U, the intra-chunk output, G: fp32
    return (size_t)B * Hv * NC * ((size_t)CK * dk * 3 + (size_t)CK * dv * 2 + CK) * sizeof(float);
}

bool delta_chunked_supported(int dk, int dv) { return dk == 128 && dv == 128; }

hipError_t launch_delta_chunked(const DeltaArgs& a, int dk, int dv, void* workspace, size_t ws_bytes,
                                hipStream_t stream) {
    if (!delta_chunked_supported(dk, dv)) return hipErrorInvalidValue;
    if (a.B <= 0 || a.T <= 0) return hipSuccess;
    if (!workspace || ws_bytes < delta_chunked_workspace(a.B, a.T, a.Hv, dk, dv)) return hipErrorInvalidValue;
    ChunkWs ws = chunk_ws(a, workspace);
    hipLaunchKernelGGL((chunk_prep_kernel<128, 128, false>), dim3(a.Hv, ws.NC, a.B), dim3(512), 0, stream, a, ws,
                       FrontArgs{});
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((chunk_state_kernel<128, 128, true>), dim3(a.Hv * (128 / 16), a.B), dim3(512), 0, stream, a, ws);
    return hipGetLastError();
}

hipError_t launch_front_chunked(const FrontArgs& f, float* conv_state, int* conv_pos, const DeltaArgs& r,
                                void* workspace, size_t ws_bytes, hipStream_t stream) {
    if (!delta_chunked_supported(f.dk, f.dv) || f.B != r.B || f.T != r.T) return hipErrorInvalidValue;
    if (r.B <= 0 || r.T <= 0) return hipSuccess;
    if (!workspace || ws_bytes < delta_chunked_workspace(r.B, r.T, r.Hv, f.dk, f.dv)) return hipErrorInvalidValue;
    ChunkWs ws = chunk_ws(r, workspace);
    DeltaArgs a = r;
    a.q = a.k = a.v = a.g = a.beta = nullptr;  // computed by the prep pass
    a.normalize = 1;
    a.scale = 1.0f / std::sqrt((float)f.dk);
    hipLaunchKernelGGL((chunk_prep_kernel<128, 128, true>), dim3(a.Hv, ws.NC, a.B), dim3(512), 0, stream, a, ws, f);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // the prep pass has read the old history: roll it forward now
    e = launch_conv_commit(f.P, f.NP, f.B, f.T, f.slot_ids, f.max_slots, f.nk, f.nv, f.dk, f.dv, conv_state,
                           conv_pos, stream);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((chunk_state_kernel<128, 128, false>), dim3(a.Hv * (128 / 16), a.B), dim3(512), 0, stream, a,
                       ws);
    return hipGetLastError();
}

}  // namespace gdn

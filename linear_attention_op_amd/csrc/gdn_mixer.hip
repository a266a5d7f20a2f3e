// The Gated DeltaNet mixer between the two projections.
//
// mixer_kernel: one workgroup per (sequence, k-head group) -- k-head kh and its R = nv / nk v-heads, 256
// threads per v-head -- runs, for each token of the launch, the whole middle of the layer: causal conv1d
// (4 taps) + SiLU on the group's 2 dk + R dv channels (q and k once for the group), q/k L2 norm, the gating
// scalars, the delta-rule update of each v-head's fp32 dk x dv state and the gated RMSNorm, with the states
// held in VGPRs from the first token to the last.  A state is read from HBM once and written once per
// launch; nothing else of size dk*dv moves.  This is the decode path (and short prefills).  It restates,
// per token, wormhole_n150/qwen3.5_9B/kernels/layer_compute.cpp C1-C6 (74-395) with
// layer_reader.cpp:103-124,184-197 for the conv history; HF:432-543 for the layer math.
//
// Load order matters: vector-memory loads complete in order, so every load the first token's conv,
// norms and gating need (history, taps, the projection row, z) is issued before the 64 KB states; that
// front-end work then runs while the states are still arriving.
//
// The conv history is the k-head group's 4-entry ring (see conv_group_width in gdn_common.h): a workgroup
// reads the three window entries, slides them through registers over the tokens and writes back only the
// inputs of the last min(T, 3) tokens and its v-heads' new ring positions.  Single-token launches run one
// workgroup per v-head (twice the workgroups of a group, so two fit a CU beside each other); the group's q
// and k channels are then read by all R of its workgroups and written by the first, into the ring entry no
// window reads.  Longer launches run one workgroup per group, which owns the whole ring.
//
// conv_front_kernel / conv_commit_kernel / gated_rmsnorm_kernel: the same front end and norm split into
// token-parallel kernels for long prefills, where the recurrence runs in the chunked form.
#include "gdn_common.h"
#include "gdn_delta_core.h"

namespace gdn {

// PER_HEAD: one workgroup of 256 threads per (v-head, sequence), single-token launches only; else one of
// 256 R threads per (k-head group, sequence).  NS > 1 (PER_HEAD only): NS workgroups per (v-head,
// sequence), each owning DV / NS state columns; the recurrence is exact per column, but the gated RMSNorm
// spans the head, so these workgroups write the output and its partial sums of squares (MixerArgs::ss_part)
// and the norm runs in the out_proj (launch_out_proj_gnorm), which also advances the ring positions: a
// workgroup that advanced them here could do so before a sibling of the same head has read them.
template <int DK, int DV, int R, bool PER_HEAD, int NS = 1>
__global__ __launch_bounds__(PER_HEAD ? 256 : 256 * R) void mixer_kernel(MixerArgs a) {
    static_assert(NS == 1 || PER_HEAD, "split heads are single-token workgroups");
    constexpr int HW = PER_HEAD ? 1 : R;     // v-heads of the workgroup
    constexpr int NTH = 256 * HW;
    constexpr int DVS = DV / NS;             // state columns of the workgroup
    constexpr int CHG = 2 * DK + R * DV;     // channels of the group (a ring entry)
    constexpr int CHW = 2 * DK + HW * DVS;   // channels of the workgroup
    constexpr int CPT = (CHW + NTH - 1) / NTH;
    using Tile = DeltaTile<DK, DVS, 256, DV>;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int sub = PER_HEAD ? 0 : tid >> 8, stid = tid & 255, swave = wave & 3;  // v-head of the workgroup
    const int cs = PER_HEAD ? blockIdx.x % NS : 0, c0 = cs * DVS;  // column slice of the workgroup
    const int h = PER_HEAD ? blockIdx.x / NS : blockIdx.x * R + sub, b = blockIdx.y;
    const int kh = PER_HEAD ? blockIdx.x / NS / R : blockIdx.x;
    const int h0 = PER_HEAD ? h : kh * R;    // first v-head of the workgroup
    const int nv = a.nv, nk = a.nk;
    const int Kd = nk * DK, Vd = nv * DV, CD = 2 * Kd + Vd;
    const int slot = a.slot_ids ? a.slot_ids[b] : b;
    if ((unsigned)slot >= (unsigned)a.max_slots) return;
    const int T = PER_HEAD ? 1 : a.T;  // per-head workgroups run single-token launches only

    __shared__ float sq[DK], sk[DK], sv[HW][DVS];
    __shared__ float red[HW][4][2][DVS];

    // ---- state-independent loads first: history, taps, the first token's projection values --------
    float* hist = a.conv_state + ((size_t)slot * nk + kh) * CONV_RING * CHG;
    int* posp = a.conv_pos + (size_t)slot * nv + h0;
    const int pos = *posp;
    float hx[CPT][3], xin[CPT];
    float4 tap[CPT];
    int pcol[CPT], gch[CPT];
    const float* Prow = a.P + (size_t)b * T * a.NP;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        const int ch = tid + NTH * c;
        pcol[c] = gch[c] = 0;
        if (ch < CHW) {
            // channel of the group: q | k of kh, then the v channels of this workgroup's v-heads
            gch[c] = ch < 2 * DK ? ch : 2 * DK + (h0 - kh * R) * DV + c0 + (ch - 2 * DK);
            pcol[c] = group_col(gch[c], kh, DK, DV, R, Kd);
            tap[c] = a.conv_w[pcol[c]];
#pragma unroll
            for (int j = 0; j < 3; ++j) hx[c][j] = hist[ring_index(pos, j) * CHG + gch[c]];
            xin[c] = Prow[pcol[c]];
        }
    }
    // gating inputs a, b of row m: from P, or summed over the partial slices of the split in_proj
    // (lane q of every wave loads slice q; the slices are summed with a wave reduction)
    auto load_ab = [&](size_t m, float& av_, float& bv_) {
        if (a.ab) {
            float sa = 0.f, sb = 0.f;
            if (lane < a.ab_splits) {
                const float* r = a.ab + lane * a.ab_stride + m * 2 * nv;
                sa = r[h], sb = r[nv + h];
            }
            av_ = warp_sum(sa), bv_ = warp_sum(sb);
        } else {
            const float* r = a.P + m * a.NP + CD + Vd;
            av_ = r[h], bv_ = r[nv + h];
        }
    };
    float av = 0.f, bv = 0.f;
    // single-token launches with one workgroup per head: the a | b loads go out with the others and are
    // summed at the gating, so that the state's loads are issued without waiting for them (9B batch 8:
    // 40.4 against 40.8 us per step; the split heads measured slower this way, 36.1 against 35.4 us)
    float ra = 0.f, rb = 0.f;
    if constexpr (!PER_HEAD || NS > 1) {
        load_ab((size_t)b * T, av, bv);
    } else if (a.ab) {
        if (lane < a.ab_splits) {
            const float* r = a.ab + lane * a.ab_stride + (size_t)b * 2 * nv;
            ra = r[h], rb = r[nv + h];
        }
    } else {
        const float* r = a.P + (size_t)b * a.NP + CD + Vd;
        ra = r[h], rb = r[nv + h];
    }
    float4 zv = make_float4(0.f, 0.f, 0.f, 0.f), nw = zv;
    if (NS == 1 && stid < Tile::CG) {
        zv = *reinterpret_cast<const float4*>(Prow + CD + h * DV + c0 + 4 * stid);
        nw = *reinterpret_cast<const float4*>(a.norm_w + c0 + 4 * stid);
    }
    const float negA = a.neg_A[h], dtb = a.dt_bias[h];

    // ---- then the states ---------------------------------------------------------------------------
    float* S = a.rec_state + ((size_t)slot * nv + h) * DK * DV + c0;
    Tile st;
    st.init(stid);
    st.load(S);
    const float qscale = rsqrtf((float)DK);

    for (int t = 0; t < T; ++t) {
        const size_t m = (size_t)b * T + t;
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
            const int ch = tid + NTH * c;
            if (ch < CHW) {
                const float acc = tap[c].x * hx[c][0] + tap[c].y * hx[c][1] + tap[c].z * hx[c][2] + tap[c].w * xin[c];
                hx[c][0] = hx[c][1];
                hx[c][1] = hx[c][2];
                hx[c][2] = xin[c];
                const float out = siluf_(acc);
                if (ch < DK)
                    sq[ch] = out;
                else if (ch < 2 * DK)
                    sk[ch - DK] = out;
                else
                    (&sv[0][0])[ch - 2 * DK] = out;
            }
        }
        // next token's projection values (issued now, consumed one token later)
        float av_n = 0.f, bv_n = 0.f;
        float4 zv_n = make_float4(0.f, 0.f, 0.f, 0.f);
        if (t + 1 < T) {
            const float* Pn = Prow + (size_t)(t + 1) * a.NP;
#pragma unroll
            for (int c = 0; c < CPT; ++c)
                if (tid + NTH * c < CHW) xin[c] = Pn[pcol[c]];
            load_ab(m + 1, av_n, bv_n);
            if (stid < Tile::CG) zv_n = *reinterpret_cast<const float4*>(Pn + CD + h * DV + 4 * stid);
        }
        __syncthreads();

        // |q|^2, |k|^2 and q.k, computed by every wave (no second barrier)
        float pqq = 0.f, pkk = 0.f, pqk = 0.f;
#pragma unroll
        for (int i = lane; i < DK; i += 64) {
            const float qv = sq[i], kv = sk[i];
            pqq += qv * qv, pkk += kv * kv, pqk += qv * kv;
        }
        pqq = warp_sum(pqq), pkk = warp_sum(pkk), pqk = warp_sum(pqk);
        const float rq = rsqrtf(pqq + 1e-6f) * qscale;
        const float rk = rsqrtf(pkk + 1e-6f);
        if constexpr (PER_HEAD && NS == 1) {
            av = a.ab ? warp_sum(ra) : ra;
            bv = a.ab ? warp_sum(rb) : rb;
        }
        const float d = __expf(negA * softplusf_(av + dtb));
        const float beta = sigmoidf_(bv);
        const float4 o = st.step(sq, sk, sv[sub], red[sub], rq, rk, pqk * rq * rk, d, beta, lane, swave);

        // gated RMSNorm of this head's o on the first wave of its part (lanes < CG hold all dv columns);
        // a column slice of a split head leaves o and its sum of squares to the out_proj
        if (NS > 1 && swave == 0) {
            float ss = lane < Tile::CG ? o.x * o.x + o.y * o.y + o.z * o.z + o.w * o.w : 0.f;
            ss = warp_sum(ss);
            if (lane < Tile::CG) *reinterpret_cast<float4*>(a.o_tap + m * Vd + h * DV + c0 + 4 * lane) = o;
            if (lane == 0) a.ss_part[(m * nv + h) * NS + cs] = ss;
        } else if (swave == 0) {
            float ss = lane < Tile::CG ? o.x * o.x + o.y * o.y + o.z * o.z + o.w * o.w : 0.f;
            ss = warp_sum(ss);
            if (lane < Tile::CG) {
                const float rstd = rsqrtf(ss / (float)DV + a.eps);
                ushort4 yv;
                yv.x = f2bf(o.x * rstd * nw.x * siluf_(zv.x));
                yv.y = f2bf(o.y * rstd * nw.y * siluf_(zv.y));
                yv.z = f2bf(o.z * rstd * nw.z * siluf_(zv.z));
                yv.w = f2bf(o.w * rstd * nw.w * siluf_(zv.w));
                const size_t yo = a.y_frag ? frag_offset((int)m, h * DV + 4 * lane, Vd) : m * Vd + h * DV + 4 * lane;
                *reinterpret_cast<ushort4*>(a.y + yo) = yv;
                if (a.o_tap) *reinterpret_cast<float4*>(a.o_tap + m * Vd + h * DV + 4 * lane) = o;
            }
        }
        if (t + 1 < T) {
            __syncthreads();  // the next token rewrites sq / sk / sv / red
            av = av_n, bv = bv_n, zv = zv_n;
        }
    }

    st.store(S);
    // the ring: the window's entry j (the input at launch time T - 3 + j) goes to entry (pos + T - 3 + j) % 4
    // when it is an input of this launch; older ones are already in place.  Per head, the group's q and k
    // channels are written by its first v-head's workgroup only.
    const bool own_qk = !PER_HEAD || (h % R == 0 && cs == 0);
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        const int ch = tid + NTH * c;
        if (ch < CHW && (own_qk || ch >= 2 * DK))
#pragma unroll
            for (int j = 0; j < 3; ++j)
                if (T - 3 + j >= 0) hist[ring_put(pos, T - 3 + j) * CHG + gch[c]] = hx[c][j];
    }
    // every thread read the old position before the step's barriers
    if (NS == 1 && tid < HW) posp[tid] = (pos + T) & 3;
}

template <int DK, int DV, bool PER_HEAD, int NS = 1>
hipError_t launch_mixer_r(const MixerArgs& a, hipStream_t stream) {
    const int R = a.nv / a.nk;
    const dim3 grid(PER_HEAD ? a.nv * NS : a.nk, a.B);
    const dim3 block(PER_HEAD ? 256 : 256 * R);
    switch (R) {
        case 1: hipLaunchKernelGGL((mixer_kernel<DK, DV, 1, PER_HEAD, NS>), grid, block, 0, stream, a); break;
        case 2: hipLaunchKernelGGL((mixer_kernel<DK, DV, 2, PER_HEAD, NS>), grid, block, 0, stream, a); break;
        case 3: hipLaunchKernelGGL((mixer_kernel<DK, DV, 3, PER_HEAD, NS>), grid, block, 0, stream, a); break;
        case 4: hipLaunchKernelGGL((mixer_kernel<DK, DV, 4, PER_HEAD, NS>), grid, block, 0, stream, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int DK, int DV>
hipError_t launch_mixer_d(const MixerArgs& a, hipStream_t stream) {
    // a group's v-heads share a ring: in separate workgroups only when the launch writes the one free entry
    return a.T == 1 ? launch_mixer_r<DK, DV, true>(a, stream) : launch_mixer_r<DK, DV, false>(a, stream);
}

hipError_t launch_mixer(const MixerArgs& a, int dk, int dv, hipStream_t stream) {
    if (a.B <= 0 || a.T <= 0) return hipSuccess;
    if (a.nk <= 0 || a.nv % a.nk) return hipErrorInvalidValue;
    if (a.ss_part) {
        if (a.T != 1 || dk != 128 || dv != 128 || !a.o_tap) return hipErrorInvalidValue;
        return launch_mixer_r<128, 128, true, kMixerSplit>(a, stream);
    }
    if (dk == 128 && dv == 128) return launch_mixer_d<128, 128>(a, stream);
    if (dk == 64 && dv == 64) return launch_mixer_d<64, 64>(a, stream);
    if (dk == 32 && dv == 32) return launch_mixer_d<32, 32>(a, stream);
    return hipErrorInvalidValue;
}

// ------------------------------------------------------------------------------------------------
// Long-T front end.  Grid (ceil(T / FTB), nk + ceil(Vd / 256) + 1, B): workgroup (tb, y, b) covers tokens
// [FTB tb, FTB tb + FTB) of sequence b and, for y < nk, the q | k channels of k-head y (2 dk <= 256
// channels, L2-normalised), for nk <= y < nk + ceil(Vd / 256) a block of 256 v channels, and for the
// last y the gating scalars g, beta.  A thread owns one channel and slides its 3-input window down the
// tokens, so each projection value is read once per block (plus 3 rows of overlap).
// ------------------------------------------------------------------------------------------------
constexpr int FTB = 16;

__global__ __launch_bounds__(256) void conv_front_kernel(FrontArgs a) {
    __shared__ float part[FTB][4];  // per-token sums of squares per segment of min(dk, 64) channels
    const int tid = threadIdx.x, lane = tid & 63;
    const int T = a.T, b = blockIdx.z, y = blockIdx.y;
    const int t0 = blockIdx.x * FTB, tn = min(FTB, T - t0);
    const int slot = a.slot_ids ? a.slot_ids[b] : b;
    if ((unsigned)slot >= (unsigned)a.max_slots) return;
    const int nk = a.nk, nv = a.nv, dk = a.dk, dv = a.dv;
    const int ratio = nv / nk;
    const int Kd = nk * dk, Vd = nv * dv, CD = 2 * Kd + Vd, CH = conv_group_width(dk, dv, ratio);
    const size_t row0 = (size_t)b * T + t0;
    const int nvb = (Vd + 255) / 256;

    if (y == nk + nvb) {  // gating scalars of this token block
        for (int e = tid; e < tn * nv; e += 256) {
            const int t = e / nv, hh = e % nv;
            const float* Prow = a.P + (row0 + t) * a.NP;
            a.g[(row0 + t) * nv + hh] = a.neg_A[hh] * softplusf_(Prow[CD + Vd + hh] + a.dt_bias[hh]);
            a.beta[(row0 + t) * nv + hh] = sigmoidf_(Prow[CD + Vd + nv + hh]);
        }
        return;
    }

    // this thread's channel: projection column, and where its history lives (group, channel of the group)
    const bool isqk = y < nk;
    bool active;
    int col = 0, grp = 0, local = 0, vc = 0;
    if (isqk) {
        const int kh = y, c = tid;  // c < dk: q channel c; dk <= c < 2 dk: k channel c - dk
        active = c < 2 * dk;
        col = c < dk ? kh * dk + c : Kd + kh * dk + (c - dk);
        grp = kh, local = c;
    } else {
        vc = (y - nk) * 256 + tid;
        active = vc < Vd;
        const int hh = min(vc, Vd - 1) / dv;
        col = 2 * Kd + vc;
        grp = hh / ratio, local = 2 * dk + (hh % ratio) * dv + (vc - hh * dv);
    }
    float out[FTB];
#pragma unroll
    for (int t = 0; t < FTB; ++t) out[t] = 0.f;
    if (active) {
        const float4 w = a.conv_w[col];
        // window: inputs at t0 - 3, t0 - 2, t0 - 1 (history entries for times before 0)
        const float* hist = a.conv_state + ((size_t)slot * nk + grp) * CONV_RING * CH;
        const int pos = a.conv_pos[(size_t)slot * nv + grp * ratio];
        float xs[3];
#pragma unroll
        for (int s = 3; s >= 1; --s) {
            const int ts = t0 - s;
            xs[3 - s] = ts >= 0 ? a.P[(row0 - s) * a.NP + col] : hist[ring_index(pos, 3 + ts) * CH + local];
        }
        float x0 = xs[0], x1 = xs[1], x2 = xs[2];
#pragma unroll
        for (int t = 0; t < FTB; ++t) {
            if (t < tn) {
                const float xin = a.P[(row0 + t) * a.NP + col];
                out[t] = siluf_(w.x * x0 + w.y * x1 + w.z * x2 + w.w * xin);
                x0 = x1, x1 = x2, x2 = xin;
            }
        }
    }
    if (!isqk) {
        if (active)
#pragma unroll
            for (int t = 0; t < FTB; ++t)
                if (t < tn) a.v[(row0 + t) * Vd + vc] = out[t];
        return;
    }
    // L2 norms of q (channels 0 .. dk-1) and k (dk .. 2dk-1) per token: segments of min(dk, 64) lanes
    const int seg = dk < 64 ? dk : 64;
#pragma unroll
    for (int t = 0; t < FTB; ++t) {
        float ss = out[t] * out[t];
        for (int off = 1; off < seg; off <<= 1) ss += __shfl_xor(ss, off, 64);
        if (active && (lane % seg) == 0) part[t][tid / seg] = ss;
    }
    __syncthreads();
    if (!active) return;
    const bool isq = tid < dk;
    const int kh = y, c = isq ? tid : tid - dk;
    const int nseg = dk / seg, s0 = isq ? 0 : nseg;  // q: segments [0, nseg), k: [nseg, 2 nseg)
    const float qscale = isq ? rsqrtf((float)dk) : 1.f;
    float* dst = (isq ? a.qn : a.kn) + row0 * Kd + kh * dk + c;
#pragma unroll
    for (int t = 0; t < FTB; ++t) {
        if (t < tn) {
            float ss = 0.f;
            for (int j = 0; j < nseg; ++j) ss += part[t][s0 + j];
            dst[(size_t)t * Kd] = out[t] * rsqrtf(ss + 1e-6f) * qscale;
        }
    }
}

hipError_t launch_conv_front(const FrontArgs& a, hipStream_t stream) {
    if (a.B <= 0 || a.T <= 0) return hipSuccess;
    if (2 * a.dk > 256) return hipErrorInvalidValue;  // one q | k channel group per workgroup
    const dim3 grid((a.T + FTB - 1) / FTB, a.nk + (a.nv * a.dv + 255) / 256 + 1, a.B);
    hipLaunchKernelGGL(conv_front_kernel, grid, dim3(256), 0, stream, a);
    return hipGetLastError();
}

// One workgroup per (sequence, k-head group): the inputs of the launch's last min(T, 3) tokens into the
// group's ring, and the new ring positions of its v-heads (entries from before the launch that stay in the
// window keep their place).
__global__ __launch_bounds__(256) void conv_commit_kernel(const float* __restrict__ P, int NP, int T,
                                                          const int* __restrict__ slot_ids, int max_slots, int nk,
                                                          int nv, int dk, int dv, float* __restrict__ conv_state,
                                                          int* __restrict__ conv_pos) {
    const int kh = blockIdx.x, b = blockIdx.y;
    const int slot = slot_ids ? slot_ids[b] : b;
    if ((unsigned)slot >= (unsigned)max_slots) return;
    const int R = nv / nk, Kd = nk * dk, CH = conv_group_width(dk, dv, R);
    float* hist = conv_state + ((size_t)slot * nk + kh) * CONV_RING * CH;
    int* posp = conv_pos + (size_t)slot * nv + kh * R;  // the positions of the group's v-heads
    const int pos = *posp;
    for (int c = threadIdx.x; c < CH; c += 256) {
        const int col = group_col(c, kh, dk, dv, R, Kd);
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const int tj = T - 3 + j;
            if (tj >= 0) hist[ring_put(pos, tj) * CH + c] = P[((size_t)b * T + tj) * NP + col];
        }
    }
    __syncthreads();  // every thread has read the old position
    if (threadIdx.x < R) posp[threadIdx.x] = (pos + T) & 3;
}

hipError_t launch_conv_commit(const float* P, int NP, int B, int T, const int* slot_ids, int max_slots, int nk,
                              int nv, int dk, int dv, float* conv_state, int* conv_pos, hipStream_t stream) {
    if (B <= 0 || T <= 0) return hipSuccess;
    hipLaunchKernelGGL(conv_commit_kernel, dim3(nk, B), dim3(256), 0, stream, P, NP, T, slot_ids, max_slots, nk, nv,
                       dk, dv, conv_state, conv_pos);
    return hipGetLastError();
}

// ------------------------------------------------------------------------------------------------
// Gated RMSNorm (HF:167-184; layer_compute.cpp C6 287-395), one workgroup per token row.
// ------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void gated_rmsnorm_kernel(const float* __restrict__ o, int nv, int dv,
                                                            const float* __restrict__ z, int z_stride,
                                                            const float* __restrict__ w, float eps,
                                                            u16* __restrict__ y) {
    const int m = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int Vd = nv * dv;
    const float* orow = o + (size_t)m * Vd;
    const float* zrow = z + (size_t)m * z_stride;
    for (int h = wave; h < nv; h += 4) {
        float ss = 0.f;
        for (int i = lane; i < dv; i += 64) ss += orow[h * dv + i] * orow[h * dv + i];
        ss = warp_sum(ss);
        const float rstd = rsqrtf(ss / (float)dv + eps);
        for (int i = lane; i < dv; i += 64)
            y[(size_t)m * Vd + h * dv + i] = f2bf(orow[h * dv + i] * rstd * w[i] * siluf_(zrow[h * dv + i]));
    }
}

// The same with 16-byte accesses: a head's dv values are dv / 4 consecutive lanes (one float4 each), its
// sum of squares a shuffle over those lanes; o is read once, y written as 8-byte pieces.
template <int DV>
__global__ __launch_bounds__(256) void gated_rmsnorm4_kernel(const float* __restrict__ o, int Vd,
                                                             const float* __restrict__ z, int z_stride,
                                                             const float* __restrict__ w, float eps,
                                                             u16* __restrict__ y) {
    constexpr int TPH = DV / 4;  // lanes per head
    const int m = blockIdx.x, t = threadIdx.x;
    const float* orow = o + (size_t)m * Vd;
    const float* zrow = z + (size_t)m * z_stride;
    u16* yrow = y + (size_t)m * Vd;
    const float4 wv = *reinterpret_cast<const float4*>(w + (t % TPH) * 4);
    for (int e = 4 * t; e < Vd; e += 1024) {  // whole heads per round: Vd % dv == 0
        const float4 ov = *reinterpret_cast<const float4*>(orow + e);
        const float4 zv = *reinterpret_cast<const float4*>(zrow + e);
        float ss = ov.x * ov.x + ov.y * ov.y + ov.z * ov.z + ov.w * ov.w;
#pragma unroll
        for (int off = 1; off < TPH; off <<= 1) ss += __shfl_xor(ss, off, 64);
        const float rstd = rsqrtf(ss / (float)DV + eps);
        const float y0 = ov.x * rstd * wv.x * siluf_(zv.x), y1 = ov.y * rstd * wv.y * siluf_(zv.y);
        const float y2 = ov.z * rstd * wv.z * siluf_(zv.z), y3 = ov.w * rstd * wv.w * siluf_(zv.w);
        uint2 pk;
        pk.x = (uint32_t)__builtin_bit_cast(u16, (__bf16)y0) | ((uint32_t)__builtin_bit_cast(u16, (__bf16)y1) << 16);
        pk.y = (uint32_t)__builtin_bit_cast(u16, (__bf16)y2) | ((uint32_t)__builtin_bit_cast(u16, (__bf16)y3) << 16);
        *reinterpret_cast<uint2*>(yrow + e) = pk;
    }
}

// The same for rows of exactly RND rounds of 1024 columns (Vd = 1024 RND): every round's o and z loads are
// issued first, non-temporal (each value is read once), so that the whole row is in flight at once.
template <int DV, int RND>
__global__ __launch_bounds__(256) void gated_rmsnorm4r_kernel(const float* __restrict__ o, const float* __restrict__ z,
                                                              int z_stride, const float* __restrict__ w, float eps,
                                                              u16* __restrict__ y) {
    constexpr int TPH = DV / 4, Vd = 1024 * RND;
    const int m = blockIdx.x, t = threadIdx.x;
    const float* orow = o + (size_t)m * Vd;
    const float* zrow = z + (size_t)m * z_stride;
    u16* yrow = y + (size_t)m * Vd;
    f32x4 ov[RND], zv[RND];
#pragma unroll
    for (int i = 0; i < RND; ++i) {
        ov[i] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(orow + 4 * t + 1024 * i));
        zv[i] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(zrow + 4 * t + 1024 * i));
    }
    const float4 wv = *reinterpret_cast<const float4*>(w + (t % TPH) * 4);
#pragma unroll
    for (int i = 0; i < RND; ++i) {
        float ss = ov[i][0] * ov[i][0] + ov[i][1] * ov[i][1] + ov[i][2] * ov[i][2] + ov[i][3] * ov[i][3];
#pragma unroll
        for (int off = 1; off < TPH; off <<= 1) ss += __shfl_xor(ss, off, 64);
        const float rstd = rsqrtf(ss / (float)DV + eps);
        const float y0 = ov[i][0] * rstd * wv.x * siluf_(zv[i][0]), y1 = ov[i][1] * rstd * wv.y * siluf_(zv[i][1]);
        const float y2 = ov[i][2] * rstd * wv.z * siluf_(zv[i][2]), y3 = ov[i][3] * rstd * wv.w * siluf_(zv[i][3]);
        uint2 pk;
        pk.x = (uint32_t)__builtin_bit_cast(u16, (__bf16)y0) | ((uint32_t)__builtin_bit_cast(u16, (__bf16)y1) << 16);
        pk.y = (uint32_t)__builtin_bit_cast(u16, (__bf16)y2) | ((uint32_t)__builtin_bit_cast(u16, (__bf16)y3) << 16);
        *reinterpret_cast<uint2*>(yrow + 4 * t + 1024 * i) = pk;
    }
}

hipError_t launch_gated_rmsnorm(const float* o, int M, int nv, int dv, const float* z, int z_stride,
                                const float* w, float eps, u16* y, hipStream_t stream) {
    if (M <= 0) return hipSuccess;
    const bool vec = z_stride % 4 == 0 && ((uintptr_t)z & 15) == 0 && ((uintptr_t)o & 15) == 0 &&
                     ((uintptr_t)y & 7) == 0 && ((uintptr_t)w & 15) == 0 && (dv == 32 || dv == 64 || dv == 128);
    if (vec) {
        const int Vd = nv * dv;
        if (dv == 128 && Vd == 4096)
            hipLaunchKernelGGL((gated_rmsnorm4r_kernel<128, 4>), dim3(M), dim3(256), 0, stream, o, z, z_stride, w, eps, y);
        else if (dv == 128 && Vd == 2048)
            hipLaunchKernelGGL((gated_rmsnorm4r_kernel<128, 2>), dim3(M), dim3(256), 0, stream, o, z, z_stride, w, eps, y);
        else if (dv == 128)
            hipLaunchKernelGGL(gated_rmsnorm4_kernel<128>, dim3(M), dim3(256), 0, stream, o, Vd, z, z_stride, w, eps, y);
        else if (dv == 64)
            hipLaunchKernelGGL(gated_rmsnorm4_kernel<64>, dim3(M), dim3(256), 0, stream, o, Vd, z, z_stride, w, eps, y);
        else
            hipLaunchKernelGGL(gated_rmsnorm4_kernel<32>, dim3(M), dim3(256), 0, stream, o, Vd, z, z_stride, w, eps, y);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(gated_rmsnorm_kernel, dim3(M), dim3(256), 0, stream, o, nv, dv, z, z_stride, w, eps, y);
    return hipGetLastError();
}

// ------------------------------------------------------------------------------------------------
// Decoder RMSNorm between stacked layers (HF Qwen3_5RMSNorm, modeling_qwen3_5.py:720-734):
// y = x rsqrt(mean(x^2) + eps) (1 + w), fp32 math, bf16 in and out.  One workgroup per row; each
// thread owns 8-element pieces of the row, read once and kept in registers between the two passes.
// ------------------------------------------------------------------------------------------------
constexpr int RN_PIECES = 4;  // pieces of 8 per thread: rows up to 256 * 8 * 4 = 8192 wide

__global__ __launch_bounds__(256) void rmsnorm_rows_kernel(const u16* x, int H, const float* __restrict__ w,
                                                           float eps, u16* y) {  // y may alias x
    __shared__ float part[4];
    const int m = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const u16* xr = x + (size_t)m * H;
    u16x8 v[RN_PIECES];
    float ss = 0.f;
#pragma unroll
    for (int p = 0; p < RN_PIECES; ++p) {
        const int c = 8 * (tid + 256 * p);
        if (c < H) {
            v[p] = *reinterpret_cast<const u16x8*>(xr + c);
#pragma unroll
            for (int j = 0; j < 8; ++j) ss += bf2f(v[p][j]) * bf2f(v[p][j]);
        }
    }
    ss = warp_sum(ss);
    if (lane == 0) part[wave] = ss;
    __syncthreads();
    const float rstd = rsqrtf((part[0] + part[1] + part[2] + part[3]) / (float)H + eps);
#pragma unroll
    for (int p = 0; p < RN_PIECES; ++p) {
        const int c = 8 * (tid + 256 * p);
        if (c < H) {
            u16x8 o;
#pragma unroll
            for (int j = 0; j < 8; ++j) o[j] = f2bf(bf2f(v[p][j]) * rstd * (1.f + (w ? w[c + j] : 0.f)));
            *reinterpret_cast<u16x8*>(y + (size_t)m * H + c) = o;
        }
    }
}

hipError_t launch_rmsnorm_rows(const u16* x, int M, int H, const float* w, float eps, u16* y, hipStream_t stream) {
    if (M <= 0) return hipSuccess;
    if (H % 8 || H > 256 * 8 * RN_PIECES) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(M), dim3(256), 0, stream, x, H, w, eps, y);
    return hipGetLastError();
}

// ------------------------------------------------------------------------------------------------
// State import / export / zero.  The conv history crosses the boundary in the reference's layout and time
// order, [n, conv_dim, 3] with entry 2 the newest (9B/gdn_layer.py:147-151 keeps it per channel): export
// reads each group's ring from its position, import writes time order at ring position 0.
// ------------------------------------------------------------------------------------------------
// Group and channel of the group of HF conv channel `col` (q | k | v order).
__device__ __forceinline__ void channel_group(int col, int nk, int dk, int dv, int R, int* grp, int* local) {
    const int Kd = nk * dk;
    if (col < Kd) {
        *grp = col / dk, *local = col % dk;
    } else if (col < 2 * Kd) {
        *grp = (col - Kd) / dk, *local = dk + (col - Kd) % dk;
    } else {
        const int hh = (col - 2 * Kd) / dv;
        *grp = hh / R, *local = 2 * dk + (hh % R) * dv + (col - 2 * Kd) % dv;
    }
}

__global__ void state_export_kernel(const float* __restrict__ rec, const float* __restrict__ conv,
                                    const int* __restrict__ conv_pos, const int* __restrict__ slots, int max_slots,
                                    int nk, int nv, int dk, int dv, float* __restrict__ rec_out,
                                    float* __restrict__ conv_out) {
    const int i = blockIdx.y;
    const int slot = slots ? slots[i] : i;
    if ((unsigned)slot >= (unsigned)max_slots) return;
    const size_t rec_n = (size_t)nv * dk * dv;
    if (rec_out)
        for (size_t e = blockIdx.x * (size_t)blockDim.x + threadIdx.x; e < rec_n; e += (size_t)gridDim.x * blockDim.x)
            rec_out[(size_t)i * rec_n + e] = rec[(size_t)slot * rec_n + e];
    if (!conv_out) return;
    const int R = nv / nk, CD = 2 * nk * dk + nv * dv, CH = conv_group_width(dk, dv, R);
    for (int col = blockIdx.x * blockDim.x + threadIdx.x; col < CD; col += gridDim.x * blockDim.x) {
        int grp, local;
        channel_group(col, nk, dk, dv, R, &grp, &local);
        const float* hist = conv + ((size_t)slot * nk + grp) * CONV_RING * CH;
        const int pos = conv_pos[(size_t)slot * nv + grp * R];
        for (int j = 0; j < 3; ++j) conv_out[((size_t)i * CD + col) * 3 + j] = hist[ring_index(pos, j) * CH + local];
    }
}

__global__ void state_import_kernel(float* __restrict__ rec, float* __restrict__ conv, int* __restrict__ conv_pos,
                                    const int* __restrict__ slots, int max_slots, int nk, int nv, int dk, int dv,
                                    const float* __restrict__ rec_in, const float* __restrict__ conv_in) {
    const int i = blockIdx.y;
    const int slot = slots ? slots[i] : i;
    if ((unsigned)slot >= (unsigned)max_slots) return;
    const size_t rec_n = (size_t)nv * dk * dv;
    if (rec_in)
        for (size_t e = blockIdx.x * (size_t)blockDim.x + threadIdx.x; e < rec_n; e += (size_t)gridDim.x * blockDim.x)
            rec[(size_t)slot * rec_n + e] = rec_in[(size_t)i * rec_n + e];
    const int R = nv / nk, CD = 2 * nk * dk + nv * dv, CH = conv_group_width(dk, dv, R);
    for (int col = blockIdx.x * blockDim.x + threadIdx.x; col < CD; col += gridDim.x * blockDim.x) {
        int grp, local;
        channel_group(col, nk, dk, dv, R, &grp, &local);
        float* hist = conv + ((size_t)slot * nk + grp) * CONV_RING * CH;
        for (int j = 0; j < 3; ++j)  // time order j at position 0: entry 1 + j
            hist[ring_index(0, j) * CH + local] = conv_in ? conv_in[((size_t)i * CD + col) * 3 + j] : 0.f;
    }
    if (blockIdx.x == 0)
        for (int g = threadIdx.x; g < nv; g += blockDim.x) conv_pos[(size_t)slot * nv + g] = 0;
}

hipError_t launch_state_export(const float* rec_state, const float* conv_state, const int* conv_pos, const int* slots,
                               int n, int max_slots, int nk, int nv, int dk, int dv, float* rec_out, float* conv_out,
                               hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(state_export_kernel, dim3(64, n), dim3(256), 0, stream, rec_state, conv_state, conv_pos, slots,
                       max_slots, nk, nv, dk, dv, rec_out, conv_out);
    return hipGetLastError();
}

hipError_t launch_state_import(float* rec_state, float* conv_state, int* conv_pos, const int* slots, int n,
                               int max_slots, int nk, int nv, int dk, int dv, const float* rec_in,
                               const float* conv_in, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(state_import_kernel, dim3(64, n), dim3(256), 0, stream, rec_state, conv_state, conv_pos, slots,
                       max_slots, nk, nv, dk, dv, rec_in, conv_in);
    return hipGetLastError();
}

__global__ void state_zero_kernel(float* __restrict__ rec, float* __restrict__ conv, int* __restrict__ conv_pos,
                                  const int* __restrict__ slots, int max_slots, int nk, int nv, int dk, int dv) {
    const int i = blockIdx.y;
    const int slot = slots ? slots[i] : i;
    if ((unsigned)slot >= (unsigned)max_slots) return;
    const size_t rec_n = (size_t)nv * dk * dv;
    const size_t conv_n = (size_t)nk * CONV_RING * conv_group_width(dk, dv, nv / nk);
    for (size_t e = blockIdx.x * (size_t)blockDim.x + threadIdx.x; e < rec_n; e += (size_t)gridDim.x * blockDim.x)
        rec[(size_t)slot * rec_n + e] = 0.f;
    for (size_t e = blockIdx.x * (size_t)blockDim.x + threadIdx.x; e < conv_n; e += (size_t)gridDim.x * blockDim.x)
        conv[(size_t)slot * conv_n + e] = 0.f;
    if (blockIdx.x == 0)
        for (int g = threadIdx.x; g < nv; g += blockDim.x) conv_pos[(size_t)slot * nv + g] = 0;
}

hipError_t launch_state_zero(float* rec_state, float* conv_state, int* conv_pos, const int* slots, int n,
                             int max_slots, int nk, int nv, int dk, int dv, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(state_zero_kernel, dim3(64, n), dim3(256), 0, stream, rec_state, conv_state, conv_pos, slots,
                       max_slots, nk, nv, dk, dv);
    return hipGetLastError();
}

}  // namespace gdn

// One token of the gated delta rule on a workgroup-resident fp32 state tile (NTH threads).
//
// Thread (rg, cg) = (tid / CG, tid % CG) holds rows rg + RG*i (i < RPT) and columns 4cg..4cg+3 of the
// dk x dv state S (S[k][v], v contiguous), so a float4 load per row reads whole rows across the wave.
// Per token (wormhole_n150/qwen3.5_9B/reference.py:28-34, in the one-pass form of
// kernels/gdn_compute.cpp:9-12 that reads the old state once):
//     kS = S^T k,  qS = S^T q                    (one pass over the old state)
//     delta = beta (v - d kS)
//     o = d qS + (q.k) delta                     (= (d S + k delta^T)^T q)
//     S <- d S + k delta^T
// k and q are read from LDS and scaled by rk / rq on the fly (rq includes the dk^-0.5 query scale).
#pragma once
#include "gdn_common.h"

namespace gdn {

// LD: the row stride of the state in memory (a tile of DV columns out of LD-wide rows when DV < LD).
template <int DK, int DV, int NTH = 256, int LD = DV>
struct DeltaTile {
    static constexpr int CG = DV / 4;
    static constexpr int RG = NTH / CG;
    static constexpr int RPT = DK / RG;
    static constexpr int NWAVES = NTH / 64;
    static_assert(CG * RG == NTH && RPT * RG == DK && CG <= 64, "state tiling");

    float4 s[RPT];
    int cg, rg;

    __device__ __forceinline__ void init(int tid) {
        cg = tid % CG;
        rg = tid / CG;
    }
    // The state is streamed: read once and written once per launch, so both directions use
    // non-temporal accesses and do not displace the projection weights from the caches.  Row i of the
    // thread is at S + RG LD i (the same for every thread: a scalar base) + rg LD + 4 cg (one 32-bit offset
    // per thread), so the 16 accesses share a single address register.
    __device__ __forceinline__ void load(const float* S) {
        const unsigned off = (unsigned)(rg * LD + 4 * cg);
#pragma unroll
        for (int i = 0; i < RPT; ++i) {
            const float* row = S + (size_t)RG * LD * i;
            const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(row + off));
            s[i] = make_float4(v[0], v[1], v[2], v[3]);
        }
    }
    __device__ __forceinline__ void store(float* S) const {
        const unsigned off = (unsigned)(rg * LD + 4 * cg);
#pragma unroll
        for (int i = 0; i < RPT; ++i) {
            float* row = S + (size_t)RG * LD * i;
            const f32x4 v = {s[i].x, s[i].y, s[i].z, s[i].w};
            __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(row + off));
        }
    }

    // red: LDS scratch [NWAVES][2][DV].  Returns o for this thread's 4 columns (every thread gets its
    // columns).  Ends with the state updated; the caller must __syncthreads() before reusing sq/sk/sv/red.
    __device__ __forceinline__ float4 step(const float* sq, const float* sk, const float* sv, float (*red)[2][DV],
                                           float rq, float rk, float qk, float d, float beta, int lane, int wave) {
        float4 pk = make_float4(0.f, 0.f, 0.f, 0.f), pq = pk;
#pragma unroll
        for (int i = 0; i < RPT; ++i) {
            const float kr = sk[rg + RG * i] * rk, qr = sq[rg + RG * i] * rq;
            pk.x += s[i].x * kr, pk.y += s[i].y * kr, pk.z += s[i].z * kr, pk.w += s[i].w * kr;
            pq.x += s[i].x * qr, pq.y += s[i].y * qr, pq.z += s[i].z * qr, pq.w += s[i].w * qr;
        }
        pk.x = lane_group_sum<CG>(pk.x), pk.y = lane_group_sum<CG>(pk.y);
        pk.z = lane_group_sum<CG>(pk.z), pk.w = lane_group_sum<CG>(pk.w);
        pq.x = lane_group_sum<CG>(pq.x), pq.y = lane_group_sum<CG>(pq.y);
        pq.z = lane_group_sum<CG>(pq.z), pq.w = lane_group_sum<CG>(pq.w);
        if (lane < CG) {
            *reinterpret_cast<float4*>(&red[wave][0][4 * lane]) = pk;
            *reinterpret_cast<float4*>(&red[wave][1][4 * lane]) = pq;
        }
        __syncthreads();
        float4 kS = make_float4(0.f, 0.f, 0.f, 0.f), qS = kS;
#pragma unroll
        for (int w = 0; w < NWAVES; ++w) {
            const float4 u = *reinterpret_cast<const float4*>(&red[w][0][4 * cg]);
            const float4 q = *reinterpret_cast<const float4*>(&red[w][1][4 * cg]);
            kS.x += u.x, kS.y += u.y, kS.z += u.z, kS.w += u.w;
            qS.x += q.x, qS.y += q.y, qS.z += q.z, qS.w += q.w;
        }
        const float4 v4 = *reinterpret_cast<const float4*>(&sv[4 * cg]);
        float4 dl, o;
        dl.x = beta * (v4.x - d * kS.x), dl.y = beta * (v4.y - d * kS.y);
        dl.z = beta * (v4.z - d * kS.z), dl.w = beta * (v4.w - d * kS.w);
        o.x = d * qS.x + qk * dl.x, o.y = d * qS.y + qk * dl.y;
        o.z = d * qS.z + qk * dl.z, o.w = d * qS.w + qk * dl.w;
#pragma unroll
        for (int i = 0; i < RPT; ++i) {
            const float kr = sk[rg + RG * i] * rk;
            s[i].x = d * s[i].x + kr * dl.x, s[i].y = d * s[i].y + kr * dl.y;
            s[i].z = d * s[i].z + kr * dl.z, s[i].w = d * s[i].w + kr * dl.w;
        }
        return o;
    }
};

// |q|^2, |k|^2 and q.k of LDS vectors on waves 0-2 into out[0..2]; wave 3 is left to the caller.
template <int DK>
__device__ __forceinline__ void qk_sums(const float* sq, const float* sk, float* out, int lane, int wave) {
    if (wave < 3) {
        float p = 0.f;
        for (int i = lane; i < DK; i += 64) p += wave == 0 ? sq[i] * sq[i] : (wave == 1 ? sk[i] * sk[i] : sq[i] * sk[i]);
        p = warp_sum(p);
        if (lane == 0) out[wave] = p;
    }
}

}  // namespace gdn

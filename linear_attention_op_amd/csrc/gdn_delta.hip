// Gated delta rule on given q, k, v, g, beta (the recurrence-only op, fla layout).
//
// delta_seq_kernel: one workgroup per (sequence, v-head) walks the T tokens with the fp32 dk x dv state
// held in VGPRs (DeltaTile); it reads the state from HBM once and writes it once per launch.
// Restates wormhole_n150/qwen3.5_9B/reference.py:11-35 (l2norm 7-8, GQA repeat_interleave 21-23,
// scale 24) and the recurrence-only device op GatedDeltaRuleL1 (gated_delta_l1.py:131-272).
#include "gdn_common.h"
#include "gdn_delta_core.h"

namespace gdn {

template <int DK, int DV>
__global__ __launch_bounds__(256) void delta_seq_kernel(DeltaArgs a) {
    using Tile = DeltaTile<DK, DV>;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = blockIdx.x, b = blockIdx.y;
    const int Hk = a.Hk, Hv = a.Hv, kh = h / (Hv / Hk);
    const int slot = a.slot_ids ? a.slot_ids[b] : b;
    if ((unsigned)slot >= (unsigned)a.max_slots) return;
    const int T = a.T;

    __shared__ float sq[DK], sk[DK], sv[DV];
    __shared__ float red[4][2][DV];
    __shared__ float scal[4];

    float* S = a.state + ((size_t)slot * Hv + h) * DK * DV;
    Tile st;
    st.init(tid);
    st.load(S);

    for (int t = 0; t < T; ++t) {
        const size_t m = (size_t)b * T + t;
        for (int i = tid; i < DK; i += 256) {
            sq[i] = a.q[(m * Hk + kh) * DK + i];
            sk[i] = a.k[(m * Hk + kh) * DK + i];
        }
        for (int i = tid; i < DV; i += 256) sv[i] = a.v[(m * Hv + h) * DV + i];
        __syncthreads();
        qk_sums<DK>(sq, sk, scal, lane, wave);
        __syncthreads();
        const float rq = (a.normalize ? rsqrtf(scal[0] + 1e-6f) : 1.f) * a.scale;
        const float rk = a.normalize ? rsqrtf(scal[1] + 1e-6f) : 1.f;
        const float d = __expf(a.g[m * Hv + h]);
        const float beta = a.beta[m * Hv + h];
        const float4 o = st.step(sq, sk, sv, red, rq, rk, scal[2] * rq * rk, d, beta, lane, wave);
        if (tid < Tile::CG) *reinterpret_cast<float4*>(a.o + (m * Hv + h) * DV + 4 * tid) = o;
        __syncthreads();
    }
    st.store(S);
}

hipError_t launch_delta_seq(const DeltaArgs& a, int dk, int dv, hipStream_t stream) {
    const dim3 grid(a.Hv, a.B);
    if (dk == 128 && dv == 128)
        hipLaunchKernelGGL((delta_seq_kernel<128, 128>), grid, dim3(256), 0, stream, a);
    else if (dk == 64 && dv == 64)
        hipLaunchKernelGGL((delta_seq_kernel<64, 64>), grid, dim3(256), 0, stream, a);
    else if (dk == 32 && dv == 32)
        hipLaunchKernelGGL((delta_seq_kernel<32, 32>), grid, dim3(256), 0, stream, a);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace gdn

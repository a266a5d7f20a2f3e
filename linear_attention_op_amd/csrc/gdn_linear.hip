// Projections y[M, N] = x[M, K] . w[N, K]^T (nn.Linear with the HF [out, in] weight layout).
// Replaces the ttnn.linear call sites of the reference layer (wormhole_n150/qwen3.5_9B/gdn_layer.py:255-259
// in_proj and a/b projection, :272-276 out_proj).
//
// Weight layouts.  W_ROW is the HF row-major [N, K].  W_FRAG is the layout the layer keeps its weights in:
// [ceil(N/16)][K/32] blocks of 512 bf16, block (nt, kq) holding for lane l = 16 g + r the 8 values
// W[16 nt + r][32 kq + 8 g + j] at offset 8 l + j -- exactly the A operand of v_mfma_f32_16x16x32_bf16,
// so one fragment load is 1 KB of contiguous memory and a wave streams its rows sequentially.
// W_F8 is the same idea for E4M3 weights (the counterpart of the reference's bfloat8_b weight_dtype,
// 9B/gdn_layer.py:55,115-120): blocks of 16 rows x 64 columns, lane l = 16 g + r holding the 16 codes
// W[16 nt + r][64 kp + 32 h + 8 g + j] (h = 0, 1), i.e. the A operands of two consecutive k-steps, plus one
// fp32 scale per row applied to the finished dot product.  Codes are widened to bf16 in registers
// (v_cvt_scalef32_pk_bf16_fp8, exact), so the MFMA work is unchanged and the weight stream halves.
// W_F4 holds MXFP4 weights (the counterpart of the reference's bfloat4_b, 0.8B/gdn_l1.py:79-80): E2M1 codes
// in blocks of 16 rows x 128 columns, lane l = 16 g + r holding the 32 codes W[16 nt + r][128 kb + 32 h +
// 8 g + j] (four consecutive k-steps), and one E8M0 scale per row and 32 columns, four to a 32-bit word per
// lane; codes are widened to bf16 times their scale in registers (v_cvt_scalef32_pk_bf16_fp4, exact), so
// the weight stream is a quarter of bf16's plus 1/32 for the scales.
//
// Kernels (bf16 MFMA, fp32 accumulation):
//  * gemv_kernel (M <= 64, decode): HBM-bound weight streaming.  A workgroup owns 16 NTS rows of w; its
//    NW waves split K, each streaming W and x fragments through a register ring PD k-steps deep (no
//    barriers in the loop), then the partials are summed through LDS and written once, coalesced.
//    Activations may come in the same fragment layout (rows padded to 16 with zeros), which turns
//    every x load into 1 KB of contiguous memory as well.
//  * gemm_kernel / gemm256_kernel (M > 64, prefill): LDS-tiled GEMM on v_mfma_f32_32x32x16_bf16, 128x128
//    tiles (4 waves of 64x64, register-staged double buffering) for small problems and software-pipelined
//    256x256 tiles (8 waves of 128x64) once there are enough tiles to fill the chip;
//    tiles are rasterised per XCD in groups of 8 M-tiles so that workgroups running together on one
//    XCD share A and B tiles in its L2.
#include "gdn_common.h"

namespace gdn {

namespace {

template <int OUT>
__device__ __forceinline__ void store_out(void* y, size_t idx, float v) {
    if (OUT == OUT_F32 || OUT == OUT_F32_T)
        reinterpret_cast<float*>(y)[idx] = v;
    else
        reinterpret_cast<u16*>(y)[idx] = f2bf(v);
}

// ------------------------------------------------------------------------------------------------
// Layout conversion W_ROW -> W_FRAG (rows past N are zero).  One 16-byte piece per thread.
// ------------------------------------------------------------------------------------------------
__global__ void frag_tile_kernel(const u16* __restrict__ w, int N, int K, u16* __restrict__ wf) {
    const size_t e = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t pieces = (size_t)((N + 15) / 16) * (K / 32) * 64;
    if (e >= pieces) return;
    const int l = (int)(e % 64);
    const size_t blk = e / 64;
    const int kq = (int)(blk % (K / 32)), nt = (int)(blk / (K / 32));
    const int n = 16 * nt + (l & 15), k = 32 * kq + 8 * (l >> 4);
    u16x8 v = {};
    if (n < N) v = *reinterpret_cast<const u16x8*>(w + (size_t)n * K + k);
    *reinterpret_cast<u16x8*>(wf + e * 8) = v;
}

// ------------------------------------------------------------------------------------------------
// E4M3 weight quantizer: one workgroup per (padded) row.  scale = absmax / 448 (1 for a zero row);
// codes = e4m3_code(w / scale), written in W_F8 layout or row-major.  Rows past N: zero codes, scale 1.
// ------------------------------------------------------------------------------------------------
template <bool FRAG>
__global__ __launch_bounds__(256) void quantize_e4m3_kernel(const u16* __restrict__ w, int N, int K,
                                                            u8* __restrict__ q, float* __restrict__ scale) {
    __shared__ float part[4];
    const int n = blockIdx.x;
    const bool real = n < N;
    float m = 0.f;
    if (real)
        for (int k = threadIdx.x; k < K; k += 256) m = fmaxf(m, fabsf(bf2f(w[(size_t)n * K + k])));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, WAVE));
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3]));
    const float sc = m > 0.f ? m / 448.0f : 1.0f;
    if (threadIdx.x == 0 && real) scale[n] = sc;
    for (int k = threadIdx.x; k < K; k += 256) {
        const u8 c = real ? (u8)e4m3_code(bf2f(w[(size_t)n * K + k]) / sc) : (u8)0;
        q[FRAG ? f8_offset(n, k, K) : (size_t)n * K + k] = c;
    }
}

// MXFP4 quantizer: one workgroup per (padded) row, a thread per 32-column block: scale code from the
// block's largest magnitude, E2M1 codes of w / 2^(code - 127) (the division is exact: a power of two).
template <bool FRAG>
__global__ __launch_bounds__(256) void quantize_mxfp4_kernel(const u16* __restrict__ w, int N, int K,
                                                             u8* __restrict__ q, u8* __restrict__ scale) {
    const int n = blockIdx.x;
    const bool real = n < N;
    for (int kq = threadIdx.x; kq < (K >> 5); kq += 256) {
        float v[32];
        float m = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const u16x8 x = real ? *reinterpret_cast<const u16x8*>(w + (size_t)n * K + 32 * kq + 8 * i) : u16x8{};
#pragma unroll
            for (int j = 0; j < 8; ++j) v[8 * i + j] = bf2f(x[j]), m = fmaxf(m, fabsf(v[8 * i + j]));
        }
        const uint32_t e = mx_scale_code(m);
        uint32_t wd[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            wd[g] = 0;
#pragma unroll
            for (int j = 0; j < 8; ++j) wd[g] |= e2m1_code(ldexpf(v[8 * g + j], 127 - (int)e)) << (4 * j);
        }
        if (FRAG) {
#pragma unroll
            for (int g = 0; g < 4; ++g) *reinterpret_cast<uint32_t*>(q + f4_offset(n, 32 * kq + 8 * g, K)) = wd[g];
            scale[f4_scale_offset(n, kq, K)] = (u8)e;
        } else {
            *reinterpret_cast<u32x4*>(q + (size_t)n * (K >> 1) + 16 * kq) = u32x4{wd[0], wd[1], wd[2], wd[3]};
            scale[(size_t)n * (K >> 5) + kq] = (u8)e;
        }
    }
}

// MXINT8 quantizer: one workgroup per (padded) row, a thread per 32-column block: scale code 2^floor(log2 amax)
// (the element format's largest power of two is 1), codes i8_code(w / 2^(code - 127)) (the division is exact).
template <bool FRAG>
__global__ __launch_bounds__(256) void quantize_mxint8_kernel(const u16* __restrict__ w, int N, int K,
                                                              u8* __restrict__ q, u8* __restrict__ scale) {
    const int n = blockIdx.x;
    const bool real = n < N;
    for (int kq = threadIdx.x; kq < (K >> 5); kq += 256) {
        float v[32];
        float m = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const u16x8 x = real ? *reinterpret_cast<const u16x8*>(w + (size_t)n * K + 32 * kq + 8 * i) : u16x8{};
#pragma unroll
            for (int j = 0; j < 8; ++j) v[8 * i + j] = bf2f(x[j]), m = fmaxf(m, fabsf(v[8 * i + j]));
        }
        const uint32_t e = mx_scale_code<0>(m);
        uint32_t wd[8];
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            wd[g] = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                wd[g] |= ((uint32_t)i8_code(ldexpf(v[4 * g + j], 127 - (int)e)) & 0xffu) << (8 * j);
        }
        if (FRAG) {
            // the 8 codes of columns 32 kq + 8 g .. + 7 are 8 contiguous bytes of one lane of a W_F8-order block
#pragma unroll
            for (int g = 0; g < 4; ++g)
                *reinterpret_cast<uint2*>(q + f8_offset(n, 32 * kq + 8 * g, K)) = make_uint2(wd[2 * g], wd[2 * g + 1]);
            scale[f4_scale_offset(n, kq, K)] = (u8)e;
        } else {
            u32x4* dst = reinterpret_cast<u32x4*>(q + (size_t)n * K + 32 * kq);
            dst[0] = u32x4{wd[0], wd[1], wd[2], wd[3]};
            dst[1] = u32x4{wd[4], wd[5], wd[6], wd[7]};
            scale[(size_t)n * (K >> 5) + kq] = (u8)e;
        }
    }
}

// ------------------------------------------------------------------------------------------------
// GEMV: M <= 16 MT
// ------------------------------------------------------------------------------------------------
// Weight fragments are read once per call: non-temporal loads, so they do not evict the activations
// every workgroup re-reads.
__device__ __forceinline__ bf16x8 ldw(const u16* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const bf16x8*>(p));
}
__device__ __forceinline__ u32x4 ldw8(const u8* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// LDS floats of the cross-wave sum below: the upper half of the waves adds into the lower half first, so
// NW / 2 partial tiles are stored at once.
template <int NTS, int MT, int NW>
constexpr int gemv_red_floats() {
    return (NW > 1 ? NW / 2 : 1) * MT * 16 * (NTS * 16 + 1);
}

// Sum of the NW waves' partial tiles through LDS (`red`: gemv_red_floats() floats) and one coalesced
// write of rows [n0, n0 + 16 NTS): C element i of lane (r, g) in acc[t][mt] is w row n0 + 16 t + 4 g + i,
// x row 16 mt + r.  A non-NULL `scale` multiplies row n of w's results by scale[n].
template <int NTS, int MT, int NW, int OUT>
__device__ __forceinline__ void gemv_finish(f32x4 (&acc)[NTS][MT], float* red_lds, int M, int N,
                                            void* __restrict__ y, int ldy, int n0, const float* __restrict__ scale) {
    constexpr int BN = NTS * 16, BM = MT * 16, LD = BN + 1, HALF = NW > 1 ? NW / 2 : 1;
    float(*red)[BM][LD] = reinterpret_cast<float(*)[BM][LD]>(red_lds);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    if (NW > 1) {
        if (wave >= HALF) {
#pragma unroll
            for (int t = 0; t < NTS; ++t)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) red[wave - HALF][16 * mt + r][16 * t + 4 * g + i] = acc[t][mt][i];
        }
        __syncthreads();
        if (wave < HALF) {
#pragma unroll
            for (int t = 0; t < NTS; ++t)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[t][mt][i] += red[wave][16 * mt + r][16 * t + 4 * g + i];
        }
        __syncthreads();
    }
    if (wave < HALF) {
#pragma unroll
        for (int t = 0; t < NTS; ++t)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int i = 0; i < 4; ++i) red[wave][16 * mt + r][16 * t + 4 * g + i] = acc[t][mt][i];
    }
    __syncthreads();
    // OUT_F32_T: x rows fastest, so that a wave writes whole output rows
    constexpr bool TR = OUT == OUT_F32_T;
    for (int e = threadIdx.x; e < BM * BN; e += NW * 64) {
        const int m = TR ? e % BM : e / BN, nl = TR ? e / BM : e % BN, n = n0 + nl;
        if (m >= M || n >= N) continue;
        float s = 0.f;
#pragma unroll
        for (int wv = 0; wv < HALF; ++wv) s += red[wv][m][nl];
        if (scale) s *= scale[n];
        store_out<OUT>(y, TR ? (size_t)n * ldy + m : (size_t)m * ldy + n, s);
    }
}

// One workgroup of the GEMV: rows [n0, n0 + 16 NTS) of w (of N) against the M rows of x over the k-steps
// [kqb, kqb + kqn) of 32, written to y[m * ldy + n] (the partial sum of that K range).
template <int NTS, int MT, int NW, int PD, int OUT, int WL, int XL>
__device__ __forceinline__ void gemv_block(const u16* __restrict__ x, const u16* __restrict__ w, int M, int N, int K,
                                           void* __restrict__ y, int ldy, int n0, int kqb, int kqn, float* red) {

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int KQ = K >> 5;
    const int kq_per = (kqn + NW - 1) / NW;
    const int kq0 = kqb + min(kqn, wave * kq_per);
    const int nsteps = kqb + min(kqn, (wave + 1) * kq_per) - kq0;
    const int NT = (N + 15) >> 4;

    // fragment base pointers and per-k-step strides
    const u16* wp[NTS];
#pragma unroll
    for (int t = 0; t < NTS; ++t) {
        if (WL == W_FRAG)
            wp[t] = w + ((size_t)min((n0 >> 4) + t, NT - 1) * KQ + kq0) * 512 + lane * 8;
        else
            wp[t] = w + (size_t)min(n0 + 16 * t + r, N - 1) * K + 32 * kq0 + 8 * g;
    }
    constexpr size_t WSTEP = WL == W_FRAG ? 512 : 32;
    // x: row-major rows (zero past M), or fragment blocks (rows past M stored as zeros)
    const u16* xp[MT];
    bool xv[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        if (XL == W_FRAG) {
            xv[mt] = true;
            xp[mt] = x + ((size_t)mt * KQ + kq0) * 512 + lane * 8;
        } else {
            xv[mt] = 16 * mt + r < M;
            xp[mt] = x + (size_t)min(16 * mt + r, M - 1) * K + 32 * kq0 + 8 * g;
        }
    }
    constexpr size_t XSTEP = XL == W_FRAG ? 512 : 32;

    bf16x8 wb[PD][NTS], xb[PD][MT];
    const bf16x8 zero8 = {};
#pragma unroll
    for (int j = 0; j < PD; ++j) {
        if (j < nsteps) {
#pragma unroll
            for (int t = 0; t < NTS; ++t) wb[j][t] = ldw(wp[t] + j * WSTEP);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) xb[j][mt] = xv[mt] ? *reinterpret_cast<const bf16x8*>(xp[mt] + j * XSTEP) : zero8;
        }
    }
    f32x4 acc[NTS][MT];
#pragma unroll
    for (int t = 0; t < NTS; ++t)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[t][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int s0 = 0; s0 < nsteps; s0 += PD) {
#pragma unroll
        for (int j = 0; j < PD; ++j) {
            const int s = s0 + j;
            if (s < nsteps) {
#pragma unroll
                for (int t = 0; t < NTS; ++t)
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = mfma16(wb[j][t], xb[j][mt], acc[t][mt]);
                if (s + PD < nsteps) {
#pragma unroll
                    for (int t = 0; t < NTS; ++t) wb[j][t] = ldw(wp[t] + (size_t)(s + PD) * WSTEP);
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt)
                        xb[j][mt] = xv[mt] ? *reinterpret_cast<const bf16x8*>(xp[mt] + (size_t)(s + PD) * XSTEP) : zero8;
                }
            }
        }
    }

    gemv_finish<NTS, MT, NW, OUT>(acc, red, M, N, y, ldy, n0, nullptr);
}

// The same for one 16-row weight tile whose wave share is exactly SPW k-steps (K = 32 SPW NW): every weight
// fragment of the wave is issued before the first MFMA (a scheduling barrier keeps that order), activations
// follow through a PX-deep ring.  The whole weight stream of the workgroup is then in flight at once
// instead of a few k-steps of it.  Measured at the 9B out_proj (M = 64, N = K = 4096): 11.6-11.8 us against
// 13.5 us for the 4-deep ring.
template <int MT, int NW, int SPW, int PX, int OUT, int XL>
__device__ __forceinline__ void gemv_block_allw(const u16* __restrict__ x, const u16* __restrict__ w, int M, int N, int K,
                                                void* __restrict__ y, int ldy, int n0, float* red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int KQ = K >> 5, NT = (N + 15) >> 4;
    const int kq0 = wave * SPW;
    const u16* wp = w + ((size_t)min(n0 >> 4, NT - 1) * KQ + kq0) * 512 + lane * 8;
    bf16x8 wb[SPW];
#pragma unroll
    for (int s = 0; s < SPW; ++s) wb[s] = ldw(wp + (size_t)s * 512);
    const u16* xp[MT];
    bool xv[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        if (XL == W_FRAG) {
            xv[mt] = true;
            xp[mt] = x + ((size_t)mt * KQ + kq0) * 512 + lane * 8;
        } else {
            xv[mt] = 16 * mt + r < M;
            xp[mt] = x + (size_t)min(16 * mt + r, M - 1) * K + 32 * kq0 + 8 * g;
        }
    }
    constexpr size_t XSTEP = XL == W_FRAG ? 512 : 32;
    const bf16x8 zero8 = {};
    bf16x8 xb[PX][MT];
#pragma unroll
    for (int j = 0; j < PX; ++j)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) xb[j][mt] = xv[mt] ? *reinterpret_cast<const bf16x8*>(xp[mt] + j * XSTEP) : zero8;
    __builtin_amdgcn_sched_barrier(0);
    f32x4 acc[1][MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[0][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[0][mt] = mfma16(wb[s], xb[s % PX][mt], acc[0][mt]);
        if (s + PX < SPW)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
                xb[s % PX][mt] = xv[mt] ? *reinterpret_cast<const bf16x8*>(xp[mt] + (size_t)(s + PX) * XSTEP) : zero8;
    }
    gemv_finish<1, MT, NW, OUT>(acc, red, M, N, y, ldy, n0, nullptr);
}

// The same on W_F8 weights: a k-step of the ring is a k-pair (64 columns), one 16-byte load per row
// tile and two x fragments per row block; rows scaled by scale[n] at the end.  K % 64 == 0; the k range
// is [kpb, kpb + kpn) in k-pairs.  On W_I8 (MXINT8) weights the same codes come with a 2-byte load of the
// pair's two E8M0 scale bytes per row tile (`scale` is then the scale-code array in f4_scale_offset order),
// applied as the codes are widened; K % 128 == 0.
template <int NTS, int MT, int NW, int PD, int OUT, int XL, int WL = W_F8>
__device__ __forceinline__ void gemv_block_f8(const u16* __restrict__ x, const u8* __restrict__ w,
                                              const float* __restrict__ scale, int M, int N, int K,
                                              void* __restrict__ y, int ldy, int n0, int kpb, int kpn, float* red) {

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int KQ = K >> 5, KP = K >> 6;
    const int kp_per = (kpn + NW - 1) / NW;
    const int kp0 = kpb + min(kpn, wave * kp_per);
    const int nsteps = kpb + min(kpn, (wave + 1) * kp_per) - kp0;
    const int NT = (N + 15) >> 4;

    const u8* wp[NTS];
#pragma unroll
    for (int t = 0; t < NTS; ++t) wp[t] = w + ((size_t)min((n0 >> 4) + t, NT - 1) * KP + kp0) * 1024 + lane * 16;
    // x: the two k-steps of a pair are 512 elements apart in fragment layout, 32 row-major
    const u16* xp[MT];
    bool xv[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        if (XL == W_FRAG) {
            xv[mt] = true;
            xp[mt] = x + ((size_t)mt * KQ + 2 * kp0) * 512 + lane * 8;
        } else {
            xv[mt] = 16 * mt + r < M;
            xp[mt] = x + (size_t)min(16 * mt + r, M - 1) * K + 64 * kp0 + 8 * g;
        }
    }
    constexpr size_t XSTEP = XL == W_FRAG ? 1024 : 64, XHALF = XL == W_FRAG ? 512 : 32;

    u32x4 wb[PD][NTS];
    uint32_t ws[PD][NTS];  // W_I8: the k-pair's two scale bytes of this lane's row
    const u8* s8 = reinterpret_cast<const u8*>(scale);
    auto sload = [&](int t, int kp) -> uint32_t {
        const int tile = min((n0 >> 4) + t, NT - 1);
        return *reinterpret_cast<const u16*>(s8 + f4_scale_offset(16 * tile + r, 2 * kp, K));
    };
    bf16x8 xb[PD][MT][2];
    const bf16x8 zero8 = {};
    auto xload = [&](int j, int s) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                xb[j][mt][h] =
                    xv[mt] ? *reinterpret_cast<const bf16x8*>(xp[mt] + (size_t)s * XSTEP + h * XHALF) : zero8;
    };
#pragma unroll
    for (int j = 0; j < PD; ++j) {
        if (j < nsteps) {
#pragma unroll
            for (int t = 0; t < NTS; ++t) {
                wb[j][t] = ldw8(wp[t] + j * 1024);
                if constexpr (WL == W_I8) ws[j][t] = sload(t, kp0 + j);
            }
            xload(j, j);
        }
    }
    f32x4 acc[NTS][MT];
#pragma unroll
    for (int t = 0; t < NTS; ++t)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[t][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int s0 = 0; s0 < nsteps; s0 += PD) {
#pragma unroll
        for (int j = 0; j < PD; ++j) {
            const int s = s0 + j;
            if (s < nsteps) {
#pragma unroll
                for (int t = 0; t < NTS; ++t) {
                    bf16x8 a0, a1;
                    if constexpr (WL == W_I8)
                        i8x16_to_bf16(wb[j][t], i8_step(ws[j][t] & 0xffu), i8_step(ws[j][t] >> 8), a0, a1);
                    else
                        e4m3x16_to_bf16(wb[j][t], a0, a1);
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) {
                        acc[t][mt] = mfma16(a0, xb[j][mt][0], acc[t][mt]);
                        acc[t][mt] = mfma16(a1, xb[j][mt][1], acc[t][mt]);
                    }
                }
                if (s + PD < nsteps) {
#pragma unroll
                    for (int t = 0; t < NTS; ++t) {
                        wb[j][t] = ldw8(wp[t] + (size_t)(s + PD) * 1024);
                        if constexpr (WL == W_I8) ws[j][t] = sload(t, kp0 + s + PD);
                    }
                    xload(j, s + PD);
                }
            }
        }
    }
    gemv_finish<NTS, MT, NW, OUT>(acc, red, M, N, y, ldy, n0, WL == W_F8 ? scale : nullptr);
}

// The same on W_F4 weights: one 16-byte load per row tile covers a k-quad (4 k-steps, 128 columns) and its
// four scales one 32-bit load; x fragments one quad (4 k-steps) ahead, weights four quads ahead for small
// tiles (a wave's whole share at the 9B shape and batch <= 16, so its weight loads are all in flight at
// once) and two for the large ones (register budget).  K % 128 == 0; the k range is [kbb, kbb + kbn) in
// k-quads.
template <int NTS, int MT, int NW, int OUT, int XL>
__device__ __forceinline__ void gemv_block_f4(const u16* __restrict__ x, const u8* __restrict__ w,
                                              const uint32_t* __restrict__ sw, int M, int N, int K,
                                              void* __restrict__ y, int ldy, int n0, int kbb, int kbn, float* red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int KQ = K >> 5, KB = K >> 7;
    const int kb_per = (kbn + NW - 1) / NW;
    const int kb0 = kbb + min(kbn, wave * kb_per);
    const int nq = kbb + min(kbn, (wave + 1) * kb_per) - kb0;
    const int NT = (N + 15) >> 4;

    const u8* wp[NTS];
    const uint32_t* sp[NTS];
#pragma unroll
    for (int t = 0; t < NTS; ++t) {
        const size_t blk = (size_t)min((n0 >> 4) + t, NT - 1) * KB + kb0;
        wp[t] = w + blk * 1024 + lane * 16;
        sp[t] = sw + blk * 16 + r;
    }
    const u16* xp[MT];
    bool xv[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        if (XL == W_FRAG) {
            xv[mt] = true;
            xp[mt] = x + ((size_t)mt * KQ + 4 * kb0) * 512 + lane * 8;
        } else {
            xv[mt] = 16 * mt + r < M;
            xp[mt] = x + (size_t)min(16 * mt + r, M - 1) * K + 128 * kb0 + 8 * g;
        }
    }
    constexpr size_t XSTEP = XL == W_FRAG ? 512 : 32;

    constexpr int PQ = NTS * MT <= 4 ? 4 : 2;  // quads in flight
    u32x4 wq[PQ][NTS];
    uint32_t ws[PQ][NTS];
    bf16x8 xb[4][MT];
    const bf16x8 zero8 = {};
    auto wload = [&](int slot, int qd) {
#pragma unroll
        for (int t = 0; t < NTS; ++t) {
            wq[slot][t] = ldw8(wp[t] + (size_t)qd * 1024);
            ws[slot][t] = sp[t][(size_t)qd * 16];
        }
    };
    auto xload = [&](int h, int s) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
            xb[h][mt] = xv[mt] ? *reinterpret_cast<const bf16x8*>(xp[mt] + (size_t)s * XSTEP) : zero8;
    };
#pragma unroll
    for (int j = 0; j < PQ; ++j)
        if (j < nq) wload(j, j);
    if (nq > 0) {
#pragma unroll
        for (int h = 0; h < 4; ++h) xload(h, h);
    }
    f32x4 acc[NTS][MT];
#pragma unroll
    for (int t = 0; t < NTS; ++t)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[t][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int q0 = 0; q0 < nq; q0 += PQ) {
#pragma unroll
        for (int slot = 0; slot < PQ; ++slot) {
            const int qd = q0 + slot;
            if (qd < nq) {
#pragma unroll
                for (int h = 0; h < 4; ++h) {
#pragma unroll
                    for (int t = 0; t < NTS; ++t) {
                        const bf16x8 a =
                            e2m1x8_to_bf16(wq[slot][t][h], e8m0_value((ws[slot][t] >> (8 * h)) & 0xffu));
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt) acc[t][mt] = mfma16(a, xb[h][mt], acc[t][mt]);
                    }
                    if (qd + 1 < nq) xload(h, 4 * (qd + 1) + h);
                }
                if (qd + PQ < nq) wload(slot, qd + PQ);
            }
        }
    }
    gemv_finish<NTS, MT, NW, OUT>(acc, red, M, N, y, ldy, n0, nullptr);
}

template <int NTS, int MT, int NW, int PD, int OUT, int WL, int XL, int SPW = 0>
__global__ __launch_bounds__(NW * 64) void gemv_kernel(const u16* __restrict__ x, const void* __restrict__ w,
                                                      const float* __restrict__ scale, int M, int N, int K,
                                                      void* __restrict__ y, int ldy) {
    __shared__ float red[gemv_red_floats<NTS, MT, NW>()];
    if constexpr (SPW > 0)
        gemv_block_allw<MT, NW, SPW, 4, OUT, XL>(x, (const u16*)w, M, N, K, y, ldy, blockIdx.x * 16, red);
    else if constexpr (WL == W_F8 || WL == W_I8)
        gemv_block_f8<NTS, MT, NW, PD, OUT, XL, WL>(x, (const u8*)w, scale, M, N, K, y, ldy, blockIdx.x * NTS * 16, 0,
                                                K >> 6, red);
    else if constexpr (WL == W_F4)
        gemv_block_f4<NTS, MT, NW, OUT, XL>(x, (const u8*)w, reinterpret_cast<const uint32_t*>(scale), M, N, K, y,
                                            ldy, blockIdx.x * NTS * 16, 0, K >> 7, red);
    else
        gemv_block<NTS, MT, NW, PD, OUT, WL, XL>(x, (const u16*)w, M, N, K, y, ldy, blockIdx.x * NTS * 16, 0,
                                                 K >> 5, red);
}

// Decode out_proj of a split-head mixer launch (GnormArgs).  The workgroup forms the gated RMSNorm of the
// M <= 4 rows, y = o rsqrt(sum_head(o^2) / dv + eps) w silu(z) in bf16, into LDS: 8 columns of one head per
// thread and pass, the head's sum of squares from the mixer's per-slice partials (HF Qwen3_5RMSNormGated,
// HF:167-184, as the fused mixer computes it).  The GEMV then reads its activations from LDS.  bf16
// weights (WL = W_FRAG): each wave issues its first pass of norm inputs, then every weight fragment of its
// k-share (SPW k-steps, as gemv_block_allw), so that the norm runs while the weights arrive (vector loads
// complete in order).  E4M3 / MXFP4 / MXINT8 weights: the norm first, then the format's GEMV block on the
// LDS rows as row-major activations.  Workgroup 0 advances the ring position of every (sequence, v-head) by
// one token.
template <int NW, int SPW, int OUT, int WL>
__global__ __launch_bounds__(NW * 64) void out_proj_gnorm_kernel(GnormArgs a) {
    static_assert(kMixerSplit == 4 || kMixerSplit == 8, "the partial sums of a (row, head) as one or two float4s");
    constexpr int PD8 = 2;  // the E4M3 / MXINT8 blocks' ring (k-pairs), as gemv() runs them
    __shared__ __attribute__((aligned(16))) u16 xs[kGnormMaxM * (kGnormMaxK + 8)];
    __shared__ float red[gemv_red_floats<1, 1, NW>()];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int M = a.M, K = a.K, KQ = K >> 5, NT = (a.N + 15) >> 4;
    const int n0 = blockIdx.x * 16, kq0 = wave * SPW;
    // LDS row stride: padded for the bf16 path's fragment reads, K for the row-major reads of the others
    const int ldx = WL == W_FRAG ? kGnormMaxK + 8 : K;

    // one pass of the norm: 8 columns of one head of row e / K per thread
    struct Piece {
        float4 o0, o1, z0, z1, w0, w1, s0, s1;
    };
    auto fetch = [&](int e) {
        const int m = e / K, c = e - m * K, hh = c / a.dv;
        const float* op = a.o + (size_t)m * K + c;
        const float* zp = a.z + (size_t)m * a.ldz + c;
        const float* np = a.norm_w + (c - hh * a.dv);
        const float* sq = a.ss + ((size_t)m * a.nv + hh) * kMixerSplit;
        Piece p;
        p.o0 = *reinterpret_cast<const float4*>(op), p.o1 = *reinterpret_cast<const float4*>(op + 4);
        p.z0 = *reinterpret_cast<const float4*>(zp), p.z1 = *reinterpret_cast<const float4*>(zp + 4);
        p.w0 = *reinterpret_cast<const float4*>(np), p.w1 = *reinterpret_cast<const float4*>(np + 4);
        p.s0 = *reinterpret_cast<const float4*>(sq);
        p.s1 = kMixerSplit > 4 ? *reinterpret_cast<const float4*>(sq + 4) : float4{0.f, 0.f, 0.f, 0.f};
        return p;
    };
    auto put = [&](int e, const Piece& p) {
        const int m = e / K, c = e - m * K;
        const float ssum = p.s0.x + p.s0.y + p.s0.z + p.s0.w + (kMixerSplit > 4 ? p.s1.x + p.s1.y + p.s1.z + p.s1.w : 0.f);
        const float rstd = rsqrtf(ssum / (float)a.dv + a.eps);
        const float ov[8] = {p.o0.x, p.o0.y, p.o0.z, p.o0.w, p.o1.x, p.o1.y, p.o1.z, p.o1.w};
        const float zv[8] = {p.z0.x, p.z0.y, p.z0.z, p.z0.w, p.z1.x, p.z1.y, p.z1.z, p.z1.w};
        const float nv8[8] = {p.w0.x, p.w0.y, p.w0.z, p.w0.w, p.w1.x, p.w1.y, p.w1.z, p.w1.w};
        u16x8 yv;
#pragma unroll
        for (int j = 0; j < 8; ++j) yv[j] = f2bf(ov[j] * rstd * nv8[j] * siluf_(zv[j]));
        *reinterpret_cast<u16x8*>(&xs[m * ldx + c]) = yv;
    };
    auto advance_ring = [&]() {
        if (blockIdx.x != 0) return;
        for (int t = tid; t < M * a.nv; t += NW * 64) {
            const int b = t / a.nv, hh = t - b * a.nv;
            const int slot = a.slot_ids ? a.slot_ids[b] : b;
            if ((unsigned)slot < (unsigned)a.max_slots) {
                int* p = a.conv_pos + (size_t)slot * a.nv + hh;
                *p = (*p + 1) & 3;
            }
        }
    };

    if constexpr (WL == W_FRAG) {
        // the first pass's inputs go out before the weights; its index is clamped so that the loads need no
        // branch
        const int e0 = 8 * tid;
        const Piece first = fetch(min(e0, M * K - 8) & ~7);
        __builtin_amdgcn_sched_barrier(0);

        const u16* wp = (const u16*)a.w + ((size_t)min(n0 >> 4, NT - 1) * KQ + kq0) * 512 + lane * 8;
        bf16x8 wb[SPW];
#pragma unroll
        for (int s = 0; s < SPW; ++s) wb[s] = ldw(wp + (size_t)s * 512);

        if (e0 < M * K) put(e0, first);
        for (int e = e0 + 8 * NW * 64; e < M * K; e += 8 * NW * 64) put(e, fetch(e));
        advance_ring();
        __syncthreads();

        f32x4 acc[1][1] = {{f32x4{0.f, 0.f, 0.f, 0.f}}};
        const bf16x8 zero8 = {};
#pragma unroll
        for (int s = 0; s < SPW; ++s) {
            const bf16x8 xb = r < M ? *reinterpret_cast<const bf16x8*>(&xs[r * ldx + 32 * (kq0 + s) + 8 * g]) : zero8;
            acc[0][0] = mfma16(wb[s], xb, acc[0][0]);
        }
        gemv_finish<1, 1, NW, OUT>(acc, red, M, a.N, a.y, a.ldy, n0, nullptr);
    } else {
        // The norm's first inputs, then one 4-byte load per 128-byte line of this wave's share of the weights
        // (as the format's block splits them: a contiguous run of 1 KB blocks of tile n0 / 16), so that those
        // lines are on their way into L2 while the norm runs; the block's own loads, issued after it, find
        // them there.  The touched words feed an empty asm at the end, which keeps the loads.
        const int e0 = 8 * tid;
        const Piece first = fetch(min(e0, M * K - 8) & ~7);
        __builtin_amdgcn_sched_barrier(0);
        const int nb = WL == W_F4 ? K >> 7 : K >> 6, per = (nb + NW - 1) / NW;
        const int b0 = min(nb, wave * per), nblk = max(1, min(nb, (wave + 1) * per) - b0);
        const u8* wt = (const u8*)a.w + ((size_t)min(n0 >> 4, NT - 1) * nb + min(b0, nb - 1)) * 1024;
        const uint32_t touched = *reinterpret_cast<const uint32_t*>(wt + (size_t)min(lane, 8 * nblk - 1) * 128);
        __builtin_amdgcn_sched_barrier(0);
        if (e0 < M * K) put(e0, first);
        for (int e = e0 + 8 * NW * 64; e < M * K; e += 8 * NW * 64) put(e, fetch(e));
        advance_ring();
        __syncthreads();
        const u16* x = xs;  // the rows in LDS, row-major with stride K
        if constexpr (WL == W_F4)
            gemv_block_f4<1, 1, NW, OUT, W_ROW>(x, (const u8*)a.w, reinterpret_cast<const uint32_t*>(a.scale), M, a.N,
                                                K, a.y, a.ldy, n0, 0, K >> 7, red);
        else
            gemv_block_f8<1, 1, NW, PD8, OUT, W_ROW, WL>(x, (const u8*)a.w, a.scale, M, a.N, K, a.y, a.ldy, n0, 0,
                                                        K >> 6, red);
        asm volatile("" ::"v"(touched));
    }
}

// Decode in_proj (fragment-layout weights and activations, fp32 out), balanced over the CUs: workgroups
// [0, G) own NTS row tiles each of the first N1 rows (G = N1 / (16 NTS), chosen ~ one per CU) and write
// them to P (row stride ldp); the remaining N2 rows (the a | b projection, 64 rows at 9B) are split into
// KS k-ranges over workgroups [G, G + ceil(N2 / 16) KS), each writing its partial sums to slice ks of
// Pab [KS][M][N2], which the mixer adds up.  One launch, no tail of half-used CUs.  Activations in fragment
// layout, or row-major (XL = W_ROW, for at most 16 rows, where re-tiling them would cost a launch).
template <int NTS, int MT, int NW, int PD, int WL, int XL>
__global__ __launch_bounds__(NW * 64) void in_proj_decode_kernel(const u16* __restrict__ x, const void* __restrict__ w,
                                                                const float* __restrict__ scale,
                                                                const u16* __restrict__ w2, int M, int N1, int N2,
                                                                int K, int G, int KS, float* __restrict__ P, int ldp,
                                                                float* __restrict__ Pab) {
    // one LDS buffer for both kinds of workgroup, so that the split workgroups fit beside the others
    constexpr int R1 = gemv_red_floats<NTS, MT, NW>(), R2 = gemv_red_floats<1, MT, NW>();
    __shared__ float red[R1 > R2 ? R1 : R2];
    const int bid = blockIdx.x;
    if (bid < G) {
        if constexpr (WL == W_F8 || WL == W_I8)
            gemv_block_f8<NTS, MT, NW, PD, OUT_F32, XL, WL>(x, (const u8*)w, scale, M, N1, K, P, ldp, bid * NTS * 16, 0,
                                                       K >> 6, red);
        else if constexpr (WL == W_F4)
            gemv_block_f4<NTS, MT, NW, OUT_F32, XL>(x, (const u8*)w, reinterpret_cast<const uint32_t*>(scale), M, N1,
                                                   K, P, ldp, bid * NTS * 16, 0, K >> 7, red);
        else
            gemv_block<NTS, MT, NW, PD, OUT_F32, W_FRAG, XL>(x, (const u16*)w, M, N1, K, P, ldp, bid * NTS * 16, 0,
                                                            K >> 5, red);
    } else {
        const int e = bid - G, nt = e % ((N2 + 15) >> 4), ks = e / ((N2 + 15) >> 4);
        const int KQ = K >> 5, per = (KQ + KS - 1) / KS;
        const int kqb = min(KQ, ks * per), kqn = min(KQ, kqb + per) - kqb;
        gemv_block<1, MT, NW, PD, OUT_F32, W_FRAG, XL>(x, w2, M, N2, K, Pab + (size_t)ks * M * N2, N2, nt * 16, kqb,
                                                      kqn, red);
    }
}

// ------------------------------------------------------------------------------------------------
// GEMM: 128 x 128 x 64 block tile, 4 waves (2 x 2), 32x32x16 MFMA
// ------------------------------------------------------------------------------------------------
constexpr int TBM = 128, TBN = 128, TBK = 64, TPAD = 8, TLD = TBK + TPAD, GROUP_M = 8;

// Epilogue of both GEMMs: C of a 32x32x16 MFMA (lane l, element e -> row 8 (e / 4) + 4 (l / 32) + e % 4,
// column l % 32) at (row0, col), times scale[col] when given.
template <int OUT>
__device__ __forceinline__ void store_tile32(const f32x16& c, int row0, int col, int M, int N, void* y, int ldy,
                                             const float* __restrict__ scale) {
    if (col >= N) return;
    const float sc = scale ? scale[col] : 1.0f;
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const int row = row0 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        if (row < M) store_out<OUT>(y, (size_t)row * ldy + col, scale ? c[e] * sc : c[e]);
    }
}

template <int OUT, int WL>
__global__ __launch_bounds__(256) void gemm_kernel(const u16* __restrict__ x, const void* __restrict__ wv,
                                                   const float* __restrict__ scale, int M, int N, int K,
                                                   void* __restrict__ y, int ldy) {
    __shared__ __attribute__((aligned(16))) u16 As[2][TBM * TLD];
    __shared__ __attribute__((aligned(16))) u16 Bs[2][TBN * TLD];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    // Tile order.  The dispatcher hands workgroup ids to the 8 XCDs round-robin; give XCD x the
    // contiguous tile range [x per, (x + 1) per) and walk it in groups of GROUP_M M-tiles (M fastest),
    // so the workgroups in flight on one XCD cover a compact block of tiles and share its L2.
    const int TM = (M + TBM - 1) / TBM, TN = (N + TBN - 1) / TBN, total = TM * TN;
    const int id = blockIdx.x, per = total / 8;
    const int t = id < 8 * per ? (id % 8) * per + id / 8 : id;
    const int gsz = GROUP_M * TN;
    const int first_m = (t / gsz) * GROUP_M;
    const int gm = min(TM - first_m, GROUP_M);
    const int tm = first_m + (t % gsz) % gm, tn = (t % gsz) / gm;
    const int m0 = tm * TBM, n0 = tn * TBN;

    // global -> register staging: 1024 16-byte pieces per operand tile, 4 per thread (W_F8: 512 B pieces,
    // 2 per thread, each widened to two 16-byte bf16 pieces on the way to LDS)
    constexpr int NB = WL == W_F8 || WL == W_F4 || WL == W_I8 ? 2 : 4;
    const u16* w = (const u16*)wv;
    const u8* w8 = (const u8*)wv;
    u16x8 ra[4], rb[4];
    u32x4 rq[2];
    uint32_t rs[2];  // W_I8: the k-tile's two scale bytes of a piece's row
    const u16* ag[4];
    const u16* bg[4];
    const u8* bq[2];
    const uint32_t* bs4[2];
    int soffa[4], soffb[4];
    const int NT = (N + 15) >> 4;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int c = tid + 256 * j;
        const int row = c >> 3, col = (c & 7) * 8;
        ag[j] = x + (size_t)min(m0 + row, M - 1) * K + col;
        soffa[j] = row * TLD + col;
        if (WL == W_F8 || WL == W_I8) {
            // piece c (< 512) of the 8 W_F8 blocks (8 n-tiles x 1 k-pair): lane l of n-tile c / 64; its two
            // 8-code halves are columns 8 g and 32 + 8 g of row 16 ntl + r (W_I8: and that row's scale words)
            if (j < NB) {
                const int ntl = c >> 6, l = c & 63;
                const size_t nt = (size_t)min((n0 >> 4) + ntl, NT - 1);
                bq[j] = w8 + nt * (K >> 6) * 1024 + l * 16;
                if (WL == W_I8) bs4[j] = reinterpret_cast<const uint32_t*>(scale) + nt * (K >> 7) * 16 + (l & 15);
                soffb[2 * j] = (16 * ntl + (l & 15)) * TLD + 8 * (l >> 4);
                soffb[2 * j + 1] = soffb[2 * j] + 32;
            }
        } else if (WL == W_F4) {
            // piece c (< 512) of the 8 W_F4 blocks (8 n-tiles x 1 k-quad) holding this k-tile: 8 bytes of lane
            // l, the two k-steps of the tile, into the same places as a W_F8 piece; its row's scale word
            if (j < NB) {
                const int ntl = c >> 6, l = c & 63;
                const size_t blk = (size_t)min((n0 >> 4) + ntl, NT - 1) * (K >> 7);
                bq[j] = w8 + blk * 1024 + l * 16;
                bs4[j] = reinterpret_cast<const uint32_t*>(scale) + blk * 16 + (l & 15);
                soffb[2 * j] = (16 * ntl + (l & 15)) * TLD + 8 * (l >> 4);
                soffb[2 * j + 1] = soffb[2 * j] + 32;
            }
        } else if (WL == W_FRAG) {
            // piece c of the 16 fragment blocks (8 n-tiles x 2 k-steps) covering this 128 x 64 tile
            const int blk = c >> 6, l = c & 63;
            const int ntl = blk >> 1, kql = blk & 1;
            bg[j] = w + ((size_t)min((n0 >> 4) + ntl, NT - 1) * (K >> 5) + kql) * 512 + l * 8;
            soffb[j] = (16 * ntl + (l & 15)) * TLD + 32 * kql + 8 * (l >> 4);
        } else {
            bg[j] = w + (size_t)min(n0 + row, N - 1) * K + col;
            soffb[j] = row * TLD + col;
        }
    }
    // k advance per 64-wide step: row-major 64 elements, fragment layout 2 blocks, W_F8 one block (bytes)
    constexpr size_t BSTEP = WL == W_ROW ? TBK : 1024;
    auto bload = [&](int kt) {
        if constexpr (WL == W_F8 || WL == W_I8) {
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                rq[j] = *reinterpret_cast<const u32x4*>(bq[j] + (size_t)kt * BSTEP);
                if constexpr (WL == W_I8) rs[j] = bs4[j][(size_t)(kt >> 1) * 16] >> (16 * (kt & 1));
            }
        } else if constexpr (WL == W_F4) {
            // codes, and the scale word shifted so that its bytes 0, 1 belong to this k-tile's k-steps
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                const uint2 c = *reinterpret_cast<const uint2*>(bq[j] + (size_t)(kt >> 1) * 1024 + (kt & 1) * 8);
                rq[j] = u32x4{c.x, c.y, bs4[j][(size_t)(kt >> 1) * 16] >> (16 * (kt & 1)), 0u};
            }
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) rb[j] = *reinterpret_cast<const u16x8*>(bg[j] + (size_t)kt * BSTEP);
        }
    };
    auto bstore = [&](int buf) {
        if constexpr (WL == W_F8 || WL == W_I8) {
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                bf16x8 lo, hi;
                if constexpr (WL == W_I8)
                    i8x16_to_bf16(rq[j], i8_step(rs[j] & 0xffu), i8_step((rs[j] >> 8) & 0xffu), lo, hi);
                else
                    e4m3x16_to_bf16(rq[j], lo, hi);
                *reinterpret_cast<bf16x8*>(&Bs[buf][soffb[2 * j]]) = lo;
                *reinterpret_cast<bf16x8*>(&Bs[buf][soffb[2 * j + 1]]) = hi;
            }
        } else if constexpr (WL == W_F4) {
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                *reinterpret_cast<bf16x8*>(&Bs[buf][soffb[2 * j]]) =
                    e2m1x8_to_bf16(rq[j][0], e8m0_value(rq[j][2] & 0xffu));
                *reinterpret_cast<bf16x8*>(&Bs[buf][soffb[2 * j + 1]]) =
                    e2m1x8_to_bf16(rq[j][1], e8m0_value((rq[j][2] >> 8) & 0xffu));
            }
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) *reinterpret_cast<u16x8*>(&Bs[buf][soffb[j]]) = rb[j];
        }
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    const int nk = K / TBK;
#pragma unroll
    for (int j = 0; j < 4; ++j) ra[j] = *reinterpret_cast<const u16x8*>(ag[j]);
    bload(0);
#pragma unroll
    for (int j = 0; j < 4; ++j) *reinterpret_cast<u16x8*>(&As[0][soffa[j]]) = ra[j];
    bstore(0);
    __syncthreads();

    const int fr = lane & 31;
    const int fk = (lane >> 5) * 8;
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < nk) {
#pragma unroll
            for (int j = 0; j < 4; ++j) ra[j] = *reinterpret_cast<const u16x8*>(ag[j] + (size_t)(kt + 1) * TBK);
            bload(kt + 1);
        }
#pragma unroll
        for (int kk = 0; kk < TBK; kk += 16) {
            bf16x8 a[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                a[i] = *reinterpret_cast<const bf16x8*>(&As[cur][(wm * 64 + i * 32 + fr) * TLD + kk + fk]);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                b[j] = *reinterpret_cast<const bf16x8*>(&Bs[cur][(wn * 64 + j * 32 + fr) * TLD + kk + fk]);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = mfma32(a[i], b[j], acc[i][j]);
        }
        if (kt + 1 < nk) {
#pragma unroll
            for (int j = 0; j < 4; ++j) *reinterpret_cast<u16x8*>(&As[cur ^ 1][soffa[j]]) = ra[j];
            bstore(cur ^ 1);
        }
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
            store_tile32<OUT>(acc[i][j], m0 + wm * 64 + i * 32, n0 + wn * 64 + j * 32 + (lane & 31), M, N, y, ldy,
                              WL == W_F8 ? scale : nullptr);
}


// ------------------------------------------------------------------------------------------------
// Large GEMM: 256 x 256 x 64 block tile on 8 waves (2 along M x 4 along N) of 128 x 64 (4 x 2 tiles of
// 32x32x16 MFMA), two waves per SIMD so that one computes while the other waits; software-pipelined:
//  * two register staging sets: the global loads of k-tile kt + 2 are issued while tile kt is computed
//    and tile kt + 1 (loaded one step earlier) is stored to the other LDS buffer;
//  * LDS rows padded to 72 bf16 (conflict-free 16-byte fragment reads), double-buffered (147 KB);
//  * in each k-tile the fragment reads of the next k-16 sub-step, the global loads and the LDS stores are
//    threaded between the 32 MFMAs (scheduling groups), and the tile ends with an LDS-only barrier, so
//    global loads stay in flight across it.
// Measured at M = 16384, K = 4096: N = 12352 1.46 ms (1.13 PFLOP/s), N = 4096 0.47 ms, against 1.81 and
// 0.52 ms for 4 waves of 128 x 128 on the same data (same sums, bit for bit).
// The main loop is branch-free (loads past the last k-tile re-read it); K % 128 == 0.
// ------------------------------------------------------------------------------------------------
constexpr int LBM = 256, LBN = 256, LBK = 64, LLD = LBK + 8;

__device__ __forceinline__ int lds_off(int row, int ch) { return row * LLD + (ch << 3); }

template <int OUT, int WL>
__global__ __launch_bounds__(512, 1) void gemm256_kernel(const u16* __restrict__ x, const void* __restrict__ wv,
                                                         const float* __restrict__ scale, int M, int N, int K,
                                                         void* __restrict__ y, int ldy) {
    __shared__ __attribute__((aligned(16))) u16 As[2][LBM * LLD];
    __shared__ __attribute__((aligned(16))) u16 Bs[2][LBN * LLD];
    constexpr int WNW = 4, FA = 4, FB = 2;  // waves along N; 32-row fragments per wave along M and N

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WNW, wn = wave % WNW;

    const int TM = (M + LBM - 1) / LBM, TN = (N + LBN - 1) / LBN, total = TM * TN;
    const int id = blockIdx.x, per = total / 8;
    const int t = id < 8 * per ? (id % 8) * per + id / 8 : id;
    const int gsz = GROUP_M * TN;
    const int first_m = (t / gsz) * GROUP_M;
    const int gm = min(TM - first_m, GROUP_M);
    const int tm = first_m + (t % gsz) % gm, tn = (t % gsz) / gm;
    const int m0 = tm * LBM, n0 = tn * LBN;
    const int KQ = K >> 5, NT = (N + 15) >> 4;

    // staging: 4 A and 4 B pieces of 16 bytes per thread and k-tile (W_F8: 2 B pieces of 16 codes, each
    // widened to two bf16 pieces on the way to LDS)
    constexpr int NB = WL == W_F8 || WL == W_F4 || WL == W_I8 ? 2 : 4;
    const u16* w = (const u16*)wv;
    const u8* w8 = (const u8*)wv;
    const u16* ag[4];
    const u16* bg[4];
    const u8* bq[2];
    const uint32_t* bs4[2];
    int sa[4], sb[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int c = tid + 512 * j;
        const int row = c >> 3, ch = c & 7;
        ag[j] = x + (size_t)min(m0 + row, M - 1) * K + ch * 8;
        sa[j] = lds_off(row, ch);
        if (WL == W_F8 || WL == W_I8) {  // piece c (< 1024) of the 16 W_F8 blocks (16 n-tiles x 1 k-pair)
            if (j < NB) {
                const int ntl = c >> 6, l = c & 63;
                const size_t nt = (size_t)min((n0 >> 4) + ntl, NT - 1);
                bq[j] = w8 + nt * (K >> 6) * 1024 + l * 16;
                if (WL == W_I8) bs4[j] = reinterpret_cast<const uint32_t*>(scale) + nt * (K >> 7) * 16 + (l & 15);
                sb[2 * j] = lds_off(16 * ntl + (l & 15), l >> 4);
                sb[2 * j + 1] = lds_off(16 * ntl + (l & 15), 4 + (l >> 4));
            }
        } else if (WL == W_F4) {  // piece c (< 1024) of the 16 W_F4 blocks (16 n-tiles x 1 k-quad): 8 bytes
            if (j < NB) {
                const int ntl = c >> 6, l = c & 63;
                const size_t blk = (size_t)min((n0 >> 4) + ntl, NT - 1) * (K >> 7);
                bq[j] = w8 + blk * 1024 + l * 16;
                bs4[j] = reinterpret_cast<const uint32_t*>(scale) + blk * 16 + (l & 15);
                sb[2 * j] = lds_off(16 * ntl + (l & 15), l >> 4);
                sb[2 * j + 1] = lds_off(16 * ntl + (l & 15), 4 + (l >> 4));
            }
        } else if (WL == W_FRAG) {  // piece c of the 32 fragment blocks (16 n-tiles x 2 k-steps) of the tile
            const int blk = c >> 6, l = c & 63;
            const int ntl = blk >> 1, kql = blk & 1;
            bg[j] = w + ((size_t)min((n0 >> 4) + ntl, NT - 1) * KQ + kql) * 512 + l * 8;
            sb[j] = lds_off(16 * ntl + (l & 15), 4 * kql + (l >> 4));
        } else {
            bg[j] = w + (size_t)min(n0 + row, N - 1) * K + ch * 8;
            sb[j] = lds_off(row, ch);
        }
    }
    // elements (W_F8: bytes) per k-tile along a B piece's stream
    constexpr int BSTEP = WL == W_ROW ? LBK : 1024;
    const int nk = K / LBK;

    // B staging: 4 bf16 pieces, or 2 code pieces in the first half of the same registers
    u16x8 ra0[4], rb0[4], ra1[4], rb1[4];
    auto gload = [&](u16x8* ra, u16x8* rb, int kt) {
        const int k = min(kt, nk - 1);
#pragma unroll
        for (int j = 0; j < 4; ++j) ra[j] = *reinterpret_cast<const u16x8*>(ag[j] + (size_t)k * LBK);
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            if constexpr (WL == W_F8 || WL == W_I8) {
                rb[j] = __builtin_bit_cast(u16x8, *reinterpret_cast<const u32x4*>(bq[j] + (size_t)k * BSTEP));
                // W_I8: the piece's two scale bytes for this k-tile ride in the unused third register
                if constexpr (WL == W_I8) rb[2][j] = (u16)(bs4[j][(size_t)(k >> 1) * 16] >> (16 * (k & 1)));
            } else if constexpr (WL == W_F4) {
                // codes, and the scale word shifted so that its bytes 0, 1 belong to this k-tile's k-steps
                const uint2 c = *reinterpret_cast<const uint2*>(bq[j] + (size_t)(k >> 1) * 1024 + (k & 1) * 8);
                rb[j] = __builtin_bit_cast(u16x8, u32x4{c.x, c.y, bs4[j][(size_t)(k >> 1) * 16] >> (16 * (k & 1)), 0u});
            } else
                rb[j] = *reinterpret_cast<const u16x8*>(bg[j] + (size_t)k * BSTEP);
        }
    };
    auto lstore = [&](const u16x8* ra, const u16x8* rb, int buf) {
#pragma unroll
        for (int j = 0; j < 4; ++j) *reinterpret_cast<u16x8*>(&As[buf][sa[j]]) = ra[j];
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            if constexpr (WL == W_F8 || WL == W_I8) {
                bf16x8 lo, hi;
                if constexpr (WL == W_I8)
                    i8x16_to_bf16(__builtin_bit_cast(u32x4, rb[j]), i8_step(rb[2][j] & 0xffu), i8_step(rb[2][j] >> 8),
                                  lo, hi);
                else
                    e4m3x16_to_bf16(__builtin_bit_cast(u32x4, rb[j]), lo, hi);
                *reinterpret_cast<bf16x8*>(&Bs[buf][sb[2 * j]]) = lo;
                *reinterpret_cast<bf16x8*>(&Bs[buf][sb[2 * j + 1]]) = hi;
            } else if constexpr (WL == W_F4) {
                const u32x4 v = __builtin_bit_cast(u32x4, rb[j]);
                *reinterpret_cast<bf16x8*>(&Bs[buf][sb[2 * j]]) = e2m1x8_to_bf16(v[0], e8m0_value(v[2] & 0xffu));
                *reinterpret_cast<bf16x8*>(&Bs[buf][sb[2 * j + 1]]) =
                    e2m1x8_to_bf16(v[1], e8m0_value((v[2] >> 8) & 0xffu));
            } else {
                *reinterpret_cast<u16x8*>(&Bs[buf][sb[j]]) = rb[j];
            }
        }
    };

    f32x16 acc[FA][FB];
#pragma unroll
    for (int i = 0; i < FA; ++i)
#pragma unroll
        for (int j = 0; j < FB; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    const int fr = lane & 31, fh = lane >> 5;
    int aoff[FA], boff[FB];
#pragma unroll
    for (int i = 0; i < FA; ++i) aoff[i] = wm * 128 + i * 32 + fr;
#pragma unroll
    for (int j = 0; j < FB; ++j) boff[j] = wn * 64 + j * 32 + fr;
    auto rdfrag = [&](int buf, int s, bf16x8* a, bf16x8* b) {
#pragma unroll
        for (int i = 0; i < FA; ++i) a[i] = *reinterpret_cast<const bf16x8*>(&As[buf][lds_off(aoff[i], 2 * s + fh)]);
#pragma unroll
        for (int j = 0; j < FB; ++j) b[j] = *reinterpret_cast<const bf16x8*>(&Bs[buf][lds_off(boff[j], 2 * s + fh)]);
    };
    auto mma = [&](const bf16x8* a, const bf16x8* b) {
#pragma unroll
        for (int i = 0; i < FA; ++i)
#pragma unroll
            for (int j = 0; j < FB; ++j) acc[i][j] = mfma32(a[i], b[j], acc[i][j]);
    };
    // one k-tile on LDS buffer `buf`, loading tile kt_ld into (ra_ld, rb_ld) and storing (ra_st, rb_st)
    // into the other buffer
    auto tile = [&](int buf, u16x8* ra_ld, u16x8* rb_ld, const u16x8* ra_st, const u16x8* rb_st, int kt_ld) {
        bf16x8 a0[FA], b0[FB], a1[FA], b1[FB];
        rdfrag(buf, 0, a0, b0);
        rdfrag(buf, 1, a1, b1);
        gload(ra_ld, rb_ld, kt_ld);
        mma(a0, b0);
        rdfrag(buf, 2, a0, b0);
        mma(a1, b1);
        rdfrag(buf, 3, a1, b1);
        lstore(ra_st, rb_st, buf ^ 1);
        mma(a0, b0);
        mma(a1, b1);
        // 6 fragment reads up front; per k-16 sub-step 8 MFMAs, the first 6 each followed by a fragment
        // read (sub-steps 0-2), the last two by two global loads (sub-steps 0-1) or an LDS store (sub-step
        // 2); in sub-step 3 the first six by an LDS store
        __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);
        for (int ss = 0; ss < 4; ++ss)
            for (int m = 0; m < 8; ++m) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                if (ss < 3 && m < 6)
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                else if (ss < 2)
                    __builtin_amdgcn_sched_group_barrier(0x020, 2, 0);
                else if ((ss == 2 && m >= 6) || (ss == 3 && m < 6))
                    __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
            }
        lds_barrier();
    };

    gload(ra0, rb0, 0);
    gload(ra1, rb1, 1);
    lstore(ra0, rb0, 0);
    __syncthreads();
    for (int kt = 0; kt < nk; kt += 2) {
        tile(0, ra0, rb0, ra1, rb1, kt + 2);
        tile(1, ra1, rb1, ra0, rb0, kt + 3);
    }

#pragma unroll
    for (int i = 0; i < FA; ++i)
#pragma unroll
        for (int j = 0; j < FB; ++j)
            store_tile32<OUT>(acc[i][j], m0 + wm * 128 + i * 32, n0 + wn * 64 + j * 32 + (lane & 31), M, N, y, ldy,
                              WL == W_F8 ? scale : nullptr);
}

// Launch arguments shared by the projection dispatchers below.
struct LinArgs {
    const void* x;
    const void* w;
    const float* scale;
    int M, N, K;
    void* y;
    int ldy, out_kind;
};

template <int NTS, int MT, int NW, int WL, int XL, int SPW>
hipError_t gemv_allw(const LinArgs& a, hipStream_t stream) {
    const dim3 grid((a.N + 15) / 16), block(NW * 64);
    if (a.out_kind == OUT_F32_T)
        hipLaunchKernelGGL((gemv_kernel<1, MT, NW, 4, OUT_F32_T, WL, XL, SPW>), grid, block, 0, stream, (const u16*)a.x, a.w,
                           a.scale, a.M, a.N, a.K, a.y, a.ldy);
    else if (a.out_kind == OUT_F32)
        hipLaunchKernelGGL((gemv_kernel<1, MT, NW, 4, OUT_F32, WL, XL, SPW>), grid, block, 0, stream, (const u16*)a.x, a.w,
                           a.scale, a.M, a.N, a.K, a.y, a.ldy);
    else
        hipLaunchKernelGGL((gemv_kernel<1, MT, NW, 4, OUT_BF16, WL, XL, SPW>), grid, block, 0, stream, (const u16*)a.x, a.w,
                           a.scale, a.M, a.N, a.K, a.y, a.ldy);
    return hipGetLastError();
}

template <int NTS, int MT, int NW, int WL, int XL>
hipError_t gemv(const LinArgs& a, hipStream_t stream) {
    constexpr int PD = WL == W_F8 || WL == W_I8 ? 2 : 4;  // an E4M3 / MXINT8 ring slot covers two k-steps
    if constexpr (NTS == 1 && WL == W_FRAG) {
        // one weight tile per workgroup: every weight fragment of a wave in flight at once when its share is
        // 8 or 16 k-steps
        const int KQ = a.K >> 5;
        if (KQ == NW * 16) return gemv_allw<1, MT, NW, WL, XL, 16>(a, stream);
        if (KQ == NW * 8) return gemv_allw<1, MT, NW, WL, XL, 8>(a, stream);
    }
    const dim3 grid((a.N + NTS * 16 - 1) / (NTS * 16));
    const dim3 block(NW * 64);
    if (a.out_kind == OUT_F32_T)
        hipLaunchKernelGGL((gemv_kernel<NTS, MT, NW, PD, OUT_F32_T, WL, XL>), grid, block, 0, stream, (const u16*)a.x,
                           a.w, a.scale, a.M, a.N, a.K, a.y, a.ldy);
    else if (a.out_kind == OUT_F32)
        hipLaunchKernelGGL((gemv_kernel<NTS, MT, NW, PD, OUT_F32, WL, XL>), grid, block, 0, stream, (const u16*)a.x,
                           a.w, a.scale, a.M, a.N, a.K, a.y, a.ldy);
    else
        hipLaunchKernelGGL((gemv_kernel<NTS, MT, NW, PD, OUT_BF16, WL, XL>), grid, block, 0, stream, (const u16*)a.x,
                           a.w, a.scale, a.M, a.N, a.K, a.y, a.ldy);
    return hipGetLastError();
}

// Shape choice: enough workgroups to spread over the 256 CUs (NTS = rows / 16 per workgroup) and
// enough waves per workgroup to keep >= 8 k-steps of 32 per wave.  Measured on the 9B shape at M = 64:
// in_proj (N 12352, K 4096) NTS 4 / NW 4, out_proj (N 4096, K 4096) NTS 1 / NW 8.
template <int MT, int WL, int XL>
hipError_t gemv_mt(const LinArgs& a, hipStream_t stream) {
    const int NT = (a.N + 15) / 16, KQ = a.K / 32;
    if (NT >= 4 * 160) {
        if (KQ >= 64) return gemv<4, MT, 4, WL, XL>(a, stream);
        return gemv<4, MT, 2, WL, XL>(a, stream);
    }
    if (NT >= 2 * 160) {
        if (KQ >= 64) return gemv<2, MT, 8, WL, XL>(a, stream);
        return gemv<2, MT, 4, WL, XL>(a, stream);
    }
    if (KQ >= 64) return gemv<1, MT, 8, WL, XL>(a, stream);
    return gemv<1, MT, 4, WL, XL>(a, stream);
}

template <int WL, int XL>
hipError_t gemv_m(const LinArgs& a, hipStream_t stream) {
    if (a.M <= 16) return gemv_mt<1, WL, XL>(a, stream);
    if (a.M <= 32) return gemv_mt<2, WL, XL>(a, stream);
    if (a.M <= 48) return gemv_mt<3, WL, XL>(a, stream);
    return gemv_mt<4, WL, XL>(a, stream);
}

template <int WL>
hipError_t linear_wl(const LinArgs& a, int xlayout, hipStream_t stream) {
    if (a.M <= 64) {
        if (xlayout == W_FRAG) return gemv_m<WL, W_FRAG>(a, stream);
        return gemv_m<WL, W_ROW>(a, stream);
    }
    if (xlayout != W_ROW) return hipErrorInvalidValue;  // the GEMM reads row-major activations
    const u16* x = (const u16*)a.x;
    if ((size_t)a.M * a.N >= (size_t)256 * 256 * 256) {  // >= one round of 256 x 256 tiles over the CUs
        const dim3 grid(((a.M + LBM - 1) / LBM) * ((a.N + LBN - 1) / LBN));
        if (a.out_kind == OUT_F32)
            hipLaunchKernelGGL((gemm256_kernel<OUT_F32, WL>), grid, dim3(512), 0, stream, x, a.w, a.scale, a.M, a.N,
                               a.K, a.y, a.ldy);
        else
            hipLaunchKernelGGL((gemm256_kernel<OUT_BF16, WL>), grid, dim3(512), 0, stream, x, a.w, a.scale, a.M,
                               a.N, a.K, a.y, a.ldy);
        return hipGetLastError();
    }
    const dim3 grid(((a.M + TBM - 1) / TBM) * ((a.N + TBN - 1) / TBN));
    if (a.out_kind == OUT_F32)
        hipLaunchKernelGGL((gemm_kernel<OUT_F32, WL>), grid, dim3(256), 0, stream, x, a.w, a.scale, a.M, a.N, a.K,
                           a.y, a.ldy);
    else
        hipLaunchKernelGGL((gemm_kernel<OUT_BF16, WL>), grid, dim3(256), 0, stream, x, a.w, a.scale, a.M, a.N, a.K,
                           a.y, a.ldy);
    return hipGetLastError();
}

}  // namespace

size_t frag_elems(int N, int K) { return (size_t)((N + 15) / 16) * 16 * K; }

hipError_t launch_quantize_e4m3(const void* w, int N, int K, u8* q, float* scale, int to_frag, hipStream_t stream) {
    if (N <= 0 || K <= 0) return hipSuccess;
    if (to_frag) {
        if (K % 64) return hipErrorInvalidValue;
        hipLaunchKernelGGL(quantize_e4m3_kernel<true>, dim3((N + 15) / 16 * 16), dim3(256), 0, stream, (const u16*)w,
                           N, K, q, scale);
    } else {
        hipLaunchKernelGGL(quantize_e4m3_kernel<false>, dim3(N), dim3(256), 0, stream, (const u16*)w, N, K, q,
                           scale);
    }
    return hipGetLastError();
}

hipError_t launch_quantize_mxfp4(const void* w, int N, int K, u8* q, u8* scale, int to_frag, hipStream_t stream) {
    if (N <= 0 || K <= 0) return hipSuccess;
    if (K % (to_frag ? 128 : 32)) return hipErrorInvalidValue;
    const int rows = to_frag ? (N + 15) / 16 * 16 : N;
    if (to_frag)
        hipLaunchKernelGGL(quantize_mxfp4_kernel<true>, dim3(rows), dim3(256), 0, stream, (const u16*)w, N, K, q, scale);
    else
        hipLaunchKernelGGL(quantize_mxfp4_kernel<false>, dim3(rows), dim3(256), 0, stream, (const u16*)w, N, K, q, scale);
    return hipGetLastError();
}

hipError_t launch_quantize_mxint8(const void* w, int N, int K, u8* q, u8* scale, int to_frag, hipStream_t stream) {
    if (N <= 0 || K <= 0) return hipSuccess;
    if (K % (to_frag ? 128 : 32)) return hipErrorInvalidValue;
    const int rows = to_frag ? (N + 15) / 16 * 16 : N;
    if (to_frag)
        hipLaunchKernelGGL(quantize_mxint8_kernel<true>, dim3(rows), dim3(256), 0, stream, (const u16*)w, N, K, q, scale);
    else
        hipLaunchKernelGGL(quantize_mxint8_kernel<false>, dim3(rows), dim3(256), 0, stream, (const u16*)w, N, K, q,
                           scale);
    return hipGetLastError();
}

template <int SPW, int WL>
void out_proj_gnorm_launch(const GnormArgs& a, int out_kind, hipStream_t stream) {
    constexpr int NW = 8;
    const dim3 grid(a.N / 16), block(NW * 64);
    if (out_kind == OUT_F32) hipLaunchKernelGGL((out_proj_gnorm_kernel<NW, SPW, OUT_F32, WL>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((out_proj_gnorm_kernel<NW, SPW, OUT_BF16, WL>), grid, block, 0, stream, a);
}

hipError_t launch_out_proj_gnorm(const GnormArgs& a, int wlayout, int out_kind, hipStream_t stream) {
    if (a.M <= 0) return hipSuccess;
    constexpr int NW = 8;
    const bool ok = a.M <= kGnormMaxM && a.K <= kGnormMaxK && a.N % 16 == 0 && a.dv % 8 == 0 && a.K % a.dv == 0 &&
                    a.K == a.nv * a.dv && a.ldz % 4 == 0 && ((uintptr_t)a.o & 15) == 0 && ((uintptr_t)a.z & 15) == 0 &&
                    ((uintptr_t)a.norm_w & 15) == 0 && ((uintptr_t)a.ss & 15) == 0 && a.conv_pos &&
                    (out_kind == OUT_F32 || out_kind == OUT_BF16);
    if (!ok) return hipErrorInvalidValue;
    const int KQ = a.K >> 5;
    switch (wlayout) {
        case W_FRAG:
            if (KQ == NW * 16) out_proj_gnorm_launch<16, W_FRAG>(a, out_kind, stream);
            else if (KQ == NW * 8) out_proj_gnorm_launch<8, W_FRAG>(a, out_kind, stream);
            else return hipErrorInvalidValue;
            break;
        case W_F8:
            if (a.K % 64 || !a.scale) return hipErrorInvalidValue;
            out_proj_gnorm_launch<1, W_F8>(a, out_kind, stream);
            break;
        case W_I8:
            if (a.K % 128 || !a.scale) return hipErrorInvalidValue;
            out_proj_gnorm_launch<1, W_I8>(a, out_kind, stream);
            break;
        case W_F4:
            if (a.K % 128 || !a.scale) return hipErrorInvalidValue;
            out_proj_gnorm_launch<1, W_F4>(a, out_kind, stream);
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_frag_tile(const void* w, int N, int K, void* wf, hipStream_t stream) {
    const size_t pieces = frag_elems(N, K) / 8;
    hipLaunchKernelGGL(frag_tile_kernel, dim3((unsigned)((pieces + 255) / 256)), dim3(256), 0, stream, (const u16*)w,
                       N, K, (u16*)wf);
    return hipGetLastError();
}

namespace {

struct DecodeArgs {
    const u16* x;
    const void* w;
    const float* scale;
    const u16* w2;
    int M, N1, N2, K, G, KS;
    float* P;
    int ldp;
    float* Pab;
};

// 8 waves per workgroup (two per SIMD) with a two-deep ring.  Measured on the 9B shape at M = 64 (with
// the split a|b workgroups): bf16 23.6 us against 23.9 us for 4 waves and a four-deep ring (bf16 needs
// <= 128 VGPRs so that the split workgroups can run beside the others), E4M3 18.8 us.  One row tile
// (M <= 16) leaves room for a four-deep ring (93 VGPRs in bf16, 120 in E4M3 and MXFP4): graph steps of
// 37.0-37.1 against 37.3-37.4 us at 9B batch 1, and 20.1-20.2 against 20.6 us at 0.8B batch 1.  MXINT8
// keeps two (four would take 142 VGPRs: its 9B batch-1 step went from 32.6-32.8 to 34.5 us).  Six deep in
// bf16 (125 VGPRs) measured mixed: 9B batch 1 35.4-35.5 against 35.6-35.7 us, batch 8 40.4-40.5 against 40.3.
template <int NTS, int MT, int WL, int XL>
void in_proj_decode_launch(const DecodeArgs& a, hipStream_t stream) {
    constexpr int NW = 8, PD = MT == 1 && WL != W_I8 ? 4 : 2;
    const dim3 grid(a.G + ((a.N2 + 15) >> 4) * a.KS), block(NW * 64);
    hipLaunchKernelGGL((in_proj_decode_kernel<NTS, MT, NW, PD, WL, XL>), grid, block, 0, stream, a.x, a.w, a.scale,
                       a.w2, a.M, a.N1, a.N2, a.K, a.G, a.KS, a.P, a.ldp, a.Pab);
}

// Row tiles per workgroup of the decode in_proj: the smallest that keeps the main workgroups within one per CU.
int in_proj_decode_tiles(int NT1) { return NT1 <= 256 ? 1 : (NT1 <= 512 ? 2 : (NT1 <= 768 ? 3 : 4)); }

template <int MT, int WL, int XL = W_FRAG>
hipError_t in_proj_decode_mt(DecodeArgs a, hipStream_t stream) {
    const int NT1 = a.N1 >> 4;
    const int nts = in_proj_decode_tiles(NT1);
    if (NT1 % nts) return hipErrorInvalidValue;
    a.G = NT1 / nts;
    switch (nts) {
        case 1: in_proj_decode_launch<1, MT, WL, XL>(a, stream); break;
        case 2: in_proj_decode_launch<2, MT, WL, XL>(a, stream); break;
        case 3: in_proj_decode_launch<3, MT, WL, XL>(a, stream); break;
        default: in_proj_decode_launch<4, MT, WL, XL>(a, stream); break;
    }
    return hipGetLastError();
}

template <int WL>
hipError_t in_proj_decode_wl(const DecodeArgs& a, int xlayout, hipStream_t stream) {
    if (xlayout == W_ROW) return in_proj_decode_mt<1, WL, W_ROW>(a, stream);  // M <= 16
    if (a.M <= 16) return in_proj_decode_mt<1, WL>(a, stream);
    if (a.M <= 32) return in_proj_decode_mt<2, WL>(a, stream);
    if (a.M <= 48) return in_proj_decode_mt<3, WL>(a, stream);
    return in_proj_decode_mt<4, WL>(a, stream);
}

}  // namespace

bool in_proj_decode_supported(int N1, int K) {
    return N1 > 0 && N1 % 16 == 0 && K % 128 == 0 && (N1 >> 4) % in_proj_decode_tiles(N1 >> 4) == 0;
}

hipError_t launch_in_proj_decode(const void* x, int xlayout, const void* w, int wlayout, const float* w_scale,
                                 const void* w2, int M, int N1, int N2, int K, float* P, int ldp, float* Pab,
                                 int ab_splits, hipStream_t stream) {
    if (M <= 0) return hipSuccess;
    if (M > 64 || N1 % 16 || ab_splits <= 0 || K % 32) return hipErrorInvalidValue;
    if (wlayout != W_FRAG && wlayout != W_F8 && wlayout != W_F4 && wlayout != W_I8) return hipErrorInvalidValue;
    if (wlayout == W_F8 && (K % 64 || !w_scale)) return hipErrorInvalidValue;
    if ((wlayout == W_F4 || wlayout == W_I8) && (K % 128 || !w_scale)) return hipErrorInvalidValue;
    if (xlayout != W_FRAG && (xlayout != W_ROW || M > 16)) return hipErrorInvalidValue;
    const DecodeArgs a{(const u16*)x, w, w_scale, (const u16*)w2, M, N1, N2, K, 0, ab_splits, P, ldp, Pab};
    if (wlayout == W_F8) return in_proj_decode_wl<W_F8>(a, xlayout, stream);
    if (wlayout == W_F4) return in_proj_decode_wl<W_F4>(a, xlayout, stream);
    if (wlayout == W_I8) return in_proj_decode_wl<W_I8>(a, xlayout, stream);
    return in_proj_decode_wl<W_FRAG>(a, xlayout, stream);
}

hipError_t launch_linear_rows_t(const void* x, const void* w, int M, int N, int K, float* y, int ldy,
                                hipStream_t stream) {
    if (M <= 0 || N <= 0) return hipSuccess;
    if (M > 64 || K % 32 || ldy < M) return hipErrorInvalidValue;
    // the GEMV's activations are the W_FRAG rows w, its streamed weights the row-major rows x
    const LinArgs a{w, x, nullptr, M, N, K, y, ldy, OUT_F32_T};
    return gemv_m<W_ROW, W_FRAG>(a, stream);
}

hipError_t launch_linear(const void* x, int xlayout, const void* w, int wlayout, const float* w_scale, int M, int N,
                         int K, void* y, int ldy, int out_kind, hipStream_t stream) {
    if (M <= 0 || N <= 0) return hipSuccess;
    if (ldy < N) return hipErrorInvalidValue;
    const LinArgs a{x, w, w_scale, M, N, K, y, ldy, out_kind};
    if (wlayout == W_F8) {
        if (K % 64 || !w_scale) return hipErrorInvalidValue;
        return linear_wl<W_F8>(a, xlayout, stream);
    }
    if (wlayout == W_F4) {
        if (K % 128 || !w_scale) return hipErrorInvalidValue;
        return linear_wl<W_F4>(a, xlayout, stream);
    }
    if (wlayout == W_I8) {
        if (K % 128 || !w_scale) return hipErrorInvalidValue;
        return linear_wl<W_I8>(a, xlayout, stream);
    }
    if (wlayout == W_FRAG) return linear_wl<W_FRAG>(a, xlayout, stream);
    return linear_wl<W_ROW>(a, xlayout, stream);
}

}  // namespace gdn

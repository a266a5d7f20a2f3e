// Projections y[M, N] = x[M, K] . w[N, K]^T (nn.Linear with the HF [out, in] weight layout).
// Replaces the ttnn.linear call sites of the reference layer (wormhole_n150/qwen3.5_9B/gdn_layer.py:255-259
// in_proj and a/b projection, :272-276 out_proj).
//
// Two kernels, both on bf16 MFMA with fp32 accumulation:
//  * linear_skinny_kernel (M <= 64, decode): HBM-bound weight streaming.  A workgroup owns NTS*16 rows
//    of w and all M rows of x; its NW waves split K, so every weight byte is read exactly once and
//    in flight from many waves at a time.  The wave partials are summed through LDS.  Both operands of
//    v_mfma_f32_16x16x32_bf16 are loaded straight from global memory: a lane holds 8 consecutive k of
//    one row, and since the MFMA sums over k, any k order shared by A and B gives the same dot product.
//  * linear_tiled_kernel (M > 64, prefill): 128x128x64 LDS-tiled GEMM on v_mfma_f32_32x32x16_bf16,
//    four waves in a 2x2 grid of 64x64 warp tiles, register-staged double buffering.
#include "gdn_common.h"

namespace gdn {

template <int OUT>
__device__ __forceinline__ void store_out(void* y, size_t idx, float v) {
    if (OUT == OUT_F32)
        reinterpret_cast<float*>(y)[idx] = v;
    else
        reinterpret_cast<u16*>(y)[idx] = f2bf(v);
}

// ------------------------------------------------------------------------------------------------
// Skinny: M <= MT * 16 <= 64
// ------------------------------------------------------------------------------------------------
template <int NTS, int MT, int NW, int OUT>
__global__ __launch_bounds__(NW * 64) void linear_skinny_kernel(const u16* __restrict__ x, const u16* __restrict__ w,
                                                                int M, int N, int K, void* __restrict__ y) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n0 = blockIdx.x * (NTS * 16);
    const int kw = K / NW;
    const int kbeg = wave * kw;
    const int r = lane & 15;
    const int g = lane >> 4;

    const u16* wp[NTS];
#pragma unroll
    for (int nt = 0; nt < NTS; ++nt) {
        const int n = min(n0 + nt * 16 + r, N - 1);
        wp[nt] = w + (size_t)n * K + kbeg + 8 * g;
    }
    const u16* xp[MT];
    bool xv[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int m = mt * 16 + r;
        xv[mt] = m < M;
        xp[mt] = x + (size_t)min(m, M - 1) * K + kbeg + 8 * g;
    }

    f32x4 acc[NTS][MT];
#pragma unroll
    for (int nt = 0; nt < NTS; ++nt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

    const bf16x8 zero8 = {};
    // main loop: 4 k-steps of 32 per iteration, all loads issued before the MFMAs that consume them
    constexpr int U = 4;
    int k = 0;
    for (; k + 32 * U <= kw; k += 32 * U) {
        bf16x8 a[U][NTS], b[U][MT];
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int nt = 0; nt < NTS; ++nt) a[u][nt] = *reinterpret_cast<const bf16x8*>(wp[nt] + k + 32 * u);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
                b[u][mt] = xv[mt] ? *reinterpret_cast<const bf16x8*>(xp[mt] + k + 32 * u) : zero8;
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int nt = 0; nt < NTS; ++nt)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = mfma16(a[u][nt], b[u][mt], acc[nt][mt]);
    }
    for (; k < kw; k += 32) {
        bf16x8 a[NTS], b[MT];
#pragma unroll
        for (int nt = 0; nt < NTS; ++nt) a[nt] = *reinterpret_cast<const bf16x8*>(wp[nt] + k);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) b[mt] = xv[mt] ? *reinterpret_cast<const bf16x8*>(xp[mt] + k) : zero8;
#pragma unroll
        for (int nt = 0; nt < NTS; ++nt)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = mfma16(a[nt], b[mt], acc[nt][mt]);
    }

    // C layout of 16x16 MFMA: lane l, element i -> row (of w) 4*(l/16) + i, column (of x) l % 16.
    constexpr int PER_WAVE = NTS * MT * 4 * 64;
    __shared__ float red[NW * PER_WAVE];
#pragma unroll
    for (int nt = 0; nt < NTS; ++nt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) red[wave * PER_WAVE + ((nt * MT + mt) * 4 + i) * 64 + lane] = acc[nt][mt][i];
    __syncthreads();

    // one output per (m, n_local); n_local fastest so the stores to y rows are contiguous
    constexpr int NL = NTS * 16;
    for (int idx = threadIdx.x; idx < MT * 16 * NL; idx += NW * 64) {
        const int nl = idx % NL;
        const int m = idx / NL;
        const int n = n0 + nl;
        if (m >= M || n >= N) continue;
        const int nt = nl >> 4, nn = nl & 15;
        const int src = ((nt * MT + (m >> 4)) * 4 + (nn & 3)) * 64 + (m & 15) + 16 * (nn >> 2);
        float s = 0.f;
#pragma unroll
        for (int wv = 0; wv < NW; ++wv) s += red[wv * PER_WAVE + src];
        store_out<OUT>(y, (size_t)m * N + n, s);
    }
}

// ------------------------------------------------------------------------------------------------
// Tiled: 128 x 128 x 64 block tile, 4 waves (2 x 2), 32x32x16 MFMA
// ------------------------------------------------------------------------------------------------
constexpr int TBM = 128, TBN = 128, TBK = 64, TPAD = 8, TLD = TBK + TPAD;

template <int OUT>
__global__ __launch_bounds__(256) void linear_tiled_kernel(const u16* __restrict__ x, const u16* __restrict__ w,
                                                           int M, int N, int K, void* __restrict__ y) {
    __shared__ __attribute__((aligned(16))) u16 As[2][TBM * TLD];
    __shared__ __attribute__((aligned(16))) u16 Bs[2][TBN * TLD];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    // Map workgroups to tiles so that consecutive workgroups (which the dispatcher spreads over the
    // 8 XCDs round-robin) walk N fastest inside a band of M tiles.
    const int tiles_n = (N + TBN - 1) / TBN;
    const int tm = blockIdx.x / tiles_n, tn = blockIdx.x % tiles_n;
    const int m0 = tm * TBM, n0 = tn * TBN;

    // global -> register staging: 1024 16-byte chunks per operand tile, 4 per thread
    u16x8 ra[4], rb[4];
    const u16* ag[4];
    const u16* bg[4];
    int soff[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int c = tid + 256 * j;
        const int row = c >> 3, col = (c & 7) * 8;
        ag[j] = x + (size_t)min(m0 + row, M - 1) * K + col;
        bg[j] = w + (size_t)min(n0 + row, N - 1) * K + col;
        soff[j] = row * TLD + col;
    }

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    const int nk = K / TBK;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        ra[j] = *reinterpret_cast<const u16x8*>(ag[j]);
        rb[j] = *reinterpret_cast<const u16x8*>(bg[j]);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        *reinterpret_cast<u16x8*>(&As[0][soff[j]]) = ra[j];
        *reinterpret_cast<u16x8*>(&Bs[0][soff[j]]) = rb[j];
    }
    __syncthreads();

    const int fr = lane & 31;
    const int fk = (lane >> 5) * 8;
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < nk) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                ra[j] = *reinterpret_cast<const u16x8*>(ag[j] + (size_t)(kt + 1) * TBK);
                rb[j] = *reinterpret_cast<const u16x8*>(bg[j] + (size_t)(kt + 1) * TBK);
            }
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
            for (int j = 0; j < 4; ++j) {
                *reinterpret_cast<u16x8*>(&As[cur ^ 1][soff[j]]) = ra[j];
                *reinterpret_cast<u16x8*>(&Bs[cur ^ 1][soff[j]]) = rb[j];
            }
        }
        __syncthreads();
    }

    // C layout of 32x32 MFMA: lane l, element e -> row 8*(e/4) + 4*(l/32) + e%4, column l % 32.
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int col = n0 + wn * 64 + j * 32 + (lane & 31);
            if (col >= N) continue;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = m0 + wm * 64 + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                if (row < M) store_out<OUT>(y, (size_t)row * N + col, acc[i][j][e]);
            }
        }
}

template <int NTS, int MT, int NW>
static hipError_t skinny(const void* x, const void* w, int M, int N, int K, void* y, int out_kind,
                         hipStream_t stream) {
    const dim3 grid((N + NTS * 16 - 1) / (NTS * 16));
    const dim3 block(NW * 64);
    if (out_kind == OUT_F32)
        hipLaunchKernelGGL((linear_skinny_kernel<NTS, MT, NW, OUT_F32>), grid, block, 0, stream,
                           (const u16*)x, (const u16*)w, M, N, K, y);
    else
        hipLaunchKernelGGL((linear_skinny_kernel<NTS, MT, NW, OUT_BF16>), grid, block, 0, stream,
                           (const u16*)x, (const u16*)w, M, N, K, y);
    return hipGetLastError();
}

template <int MT>
static hipError_t skinny_mt(const void* x, const void* w, int M, int N, int K, void* y, int out_kind,
                            hipStream_t stream) {
    // Enough workgroups to cover the 256 CUs: 32-row tiles for wide outputs, 16-row tiles otherwise.
    if (N >= 8192) return skinny<2, MT, 4>(x, w, M, N, K, y, out_kind, stream);
    return skinny<1, MT, 4>(x, w, M, N, K, y, out_kind, stream);
}

hipError_t launch_linear(const void* x, const void* w, int M, int N, int K, void* y, int out_kind,
                         hipStream_t stream) {
    if (M <= 0 || N <= 0) return hipSuccess;
    if (M <= 16) return skinny_mt<1>(x, w, M, N, K, y, out_kind, stream);
    if (M <= 32) return skinny_mt<2>(x, w, M, N, K, y, out_kind, stream);
    if (M <= 48) return skinny_mt<3>(x, w, M, N, K, y, out_kind, stream);
    if (M <= 64) return skinny_mt<4>(x, w, M, N, K, y, out_kind, stream);
    const dim3 grid(((M + TBM - 1) / TBM) * ((N + TBN - 1) / TBN));
    if (out_kind == OUT_F32)
        hipLaunchKernelGGL((linear_tiled_kernel<OUT_F32>), grid, dim3(256), 0, stream, (const u16*)x, (const u16*)w,
                           M, N, K, y);
    else
        hipLaunchKernelGGL((linear_tiled_kernel<OUT_BF16>), grid, dim3(256), 0, stream, (const u16*)x,
                           (const u16*)w, M, N, K, y);
    return hipGetLastError();
}

}  // namespace gdn

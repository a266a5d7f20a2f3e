// Projections y[M, N] = x[M, K] . w[N, K]^T (nn.Linear with the HF [out, in] weight layout).
// Replaces the ttnn.linear call sites of the reference layer (wormhole_n150/qwen3.5_9B/gdn_layer.py:255-259
// in_proj and a/b projection, :272-276 out_proj).
//
// Weight layouts.  W_ROW is the HF row-major [N, K].  W_FRAG is the layout the layer keeps its weights in:
// [ceil(N/16)][K/32] blocks of 512 bf16, block (nt, kq) holding for lane l = 16 g + r the 8 values
// W[16 nt + r][32 kq + 8 g + j] at offset 8 l + j -- exactly the A operand of v_mfma_f32_16x16x32_bf16,
// so one fragment load is 1 KB of contiguous memory and a wave streams its rows sequentially.
//
// Kernels (bf16 MFMA, fp32 accumulation):
//  * gemv_kernel (M <= 64, decode): HBM-bound weight streaming.  A workgroup owns 16 NTS rows of w; its
//    NW waves split K, each streaming W and x fragments through a register ring PD k-steps deep (no
//    barriers in the loop), then the partials are summed through LDS and written once, coalesced.
//    Activations may come in the same fragment layout (rows padded to 16 with zeros), which turns
//    every x load into 1 KB of contiguous memory as well.
//  * gemm_kernel / gemm256_kernel (M > 64, prefill): LDS-tiled GEMM on v_mfma_f32_32x32x16_bf16, 128x128
//    tiles (4 waves of 64x64, register-staged double buffering) for small problems and software-pipelined
//    256x256 tiles (4 waves of 128x128) once there are enough tiles to fill the chip;
//    tiles are rasterised per XCD in groups of 8 M-tiles so that workgroups running together on one
//    XCD share A and B tiles in its L2.
#include "gdn_common.h"

namespace gdn {

namespace {

template <int OUT>
__device__ __forceinline__ void store_out(void* y, size_t idx, float v) {
    if (OUT == OUT_F32)
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
// GEMV: M <= 16 MT
// ------------------------------------------------------------------------------------------------
// Weight fragments are read once per call: non-temporal loads, so they do not evict the activations
// every workgroup re-reads.
__device__ __forceinline__ bf16x8 ldw(const u16* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const bf16x8*>(p));
}

// One workgroup of the GEMV: rows [n0, n0 + 16 NTS) of w (of N) against the M rows of x over the k-steps
// [kqb, kqb + kqn) of 32, written to y[m * ldy + n] (the partial sum of that K range).
template <int NTS, int MT, int NW, int PD, int OUT, int WL, int XL>
__device__ __forceinline__ void gemv_block(const u16* __restrict__ x, const u16* __restrict__ w, int M, int N, int K,
                                           void* __restrict__ y, int ldy, int n0, int kqb, int kqn) {
    constexpr int BN = NTS * 16, BM = MT * 16;
    __shared__ float red[NW][BM][BN + 1];

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

    // C element i of lane (r, g) in acc[t][mt]: w row n0 + 16 t + 4 g + i, x row 16 mt + r
#pragma unroll
    for (int t = 0; t < NTS; ++t)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) red[wave][16 * mt + r][16 * t + 4 * g + i] = acc[t][mt][i];
    __syncthreads();
    for (int e = threadIdx.x; e < BM * BN; e += NW * 64) {
        const int m = e / BN, nl = e % BN, n = n0 + nl;
        if (m >= M || n >= N) continue;
        float s = 0.f;
#pragma unroll
        for (int wv = 0; wv < NW; ++wv) s += red[wv][m][nl];
        store_out<OUT>(y, (size_t)m * ldy + n, s);
    }
}

template <int NTS, int MT, int NW, int PD, int OUT, int WL, int XL>
__global__ __launch_bounds__(NW * 64) void gemv_kernel(const u16* __restrict__ x, const u16* __restrict__ w, int M,
                                                      int N, int K, void* __restrict__ y) {
    gemv_block<NTS, MT, NW, PD, OUT, WL, XL>(x, w, M, N, K, y, N, blockIdx.x * NTS * 16, 0, K >> 5);
}

// Decode in_proj (fragment-layout weights and activations, fp32 out), balanced over the CUs: workgroups
// [0, G) own NTS row tiles each of the first N1 rows (G = N1 / (16 NTS), chosen ~ one per CU) and write
// them to P (row stride ldp); the remaining N2 rows (the a | b projection, 64 rows at 9B) are split into
// KS k-ranges over workgroups [G, G + ceil(N2 / 16) KS), each writing its partial sums to slice ks of
// Pab [KS][M][N2], which the mixer adds up.  One launch, no tail of half-used CUs.
template <int NTS, int MT, int NW, int PD>
__global__ __launch_bounds__(NW * 64) void in_proj_decode_kernel(const u16* __restrict__ x, const u16* __restrict__ w,
                                                                int M, int N1, int N2, int K, int G, int KS,
                                                                float* __restrict__ P, int ldp, float* __restrict__ Pab) {
    const int bid = blockIdx.x;
    if (bid < G) {
        gemv_block<NTS, MT, NW, PD, OUT_F32, W_FRAG, W_FRAG>(x, w, M, N1, K, P, ldp, bid * NTS * 16, 0, K >> 5);
    } else {
        const int e = bid - G, nt = e % ((N2 + 15) >> 4), ks = e / ((N2 + 15) >> 4);
        const int KQ = K >> 5, per = (KQ + KS - 1) / KS;
        const int kqb = min(KQ, ks * per), kqn = min(KQ, kqb + per) - kqb;
        const u16* w2 = w + (size_t)(N1 >> 4) * KQ * 512;  // first fragment row of the split rows
        gemv_block<1, MT, NW, PD, OUT_F32, W_FRAG, W_FRAG>(x, w2, M, N2, K, Pab + (size_t)ks * M * N2, N2, nt * 16,
                                                          kqb, kqn);
    }
}

// ------------------------------------------------------------------------------------------------
// GEMM: 128 x 128 x 64 block tile, 4 waves (2 x 2), 32x32x16 MFMA
// ------------------------------------------------------------------------------------------------
constexpr int TBM = 128, TBN = 128, TBK = 64, TPAD = 8, TLD = TBK + TPAD, GROUP_M = 8;

template <int OUT, int WL>
__global__ __launch_bounds__(256) void gemm_kernel(const u16* __restrict__ x, const u16* __restrict__ w, int M, int N,
                                                   int K, void* __restrict__ y) {
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

    // global -> register staging: 1024 16-byte pieces per operand tile, 4 per thread
    u16x8 ra[4], rb[4];
    const u16* ag[4];
    const u16* bg[4];
    int soffa[4], soffb[4];
    const int NT = (N + 15) >> 4;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int c = tid + 256 * j;
        const int row = c >> 3, col = (c & 7) * 8;
        ag[j] = x + (size_t)min(m0 + row, M - 1) * K + col;
        soffa[j] = row * TLD + col;
        if (WL == W_FRAG) {
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
    // k advance per 64-wide step: row-major 64 elements, fragment layout 2 blocks
    constexpr size_t BSTEP = WL == W_FRAG ? 1024 : TBK;

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
        *reinterpret_cast<u16x8*>(&As[0][soffa[j]]) = ra[j];
        *reinterpret_cast<u16x8*>(&Bs[0][soffb[j]]) = rb[j];
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
                rb[j] = *reinterpret_cast<const u16x8*>(bg[j] + (size_t)(kt + 1) * BSTEP);
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
                *reinterpret_cast<u16x8*>(&As[cur ^ 1][soffa[j]]) = ra[j];
                *reinterpret_cast<u16x8*>(&Bs[cur ^ 1][soffb[j]]) = rb[j];
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


// ------------------------------------------------------------------------------------------------
// Large GEMM: 256 x 256 x 64 block tile, 4 waves of 128 x 128 (4 x 4 tiles of 32x32x16 MFMA, 256 fp32
// accumulators per lane in AGPRs), software-pipelined:
//  * two register staging sets: the global loads of k-tile kt + 2 are issued while tile kt is computed
//    and tile kt + 1 (loaded one step earlier) is stored to the other LDS buffer;
//  * LDS rows padded to 72 bf16 (conflict-free 16-byte fragment reads), double-buffered (147 KB);
//  * in each k-tile the fragment reads of the next k-16 sub-step, the global loads and the LDS stores are
//    threaded one by one between the 64 MFMAs (scheduling groups), and the tile ends with an LDS-only
//    barrier, so global loads stay in flight across it.
// The main loop is branch-free (loads past the last k-tile re-read it); K % 128 == 0.
// ------------------------------------------------------------------------------------------------
constexpr int LBM = 256, LBN = 256, LBK = 64, LLD = LBK + 8;

__device__ __forceinline__ int lds_off(int row, int ch) { return row * LLD + (ch << 3); }

template <int OUT, int WL>
__global__ __launch_bounds__(256, 1) void gemm256_kernel(const u16* __restrict__ x, const u16* __restrict__ w, int M,
                                                         int N, int K, void* __restrict__ y) {
    __shared__ __attribute__((aligned(16))) u16 As[2][LBM * LLD];
    __shared__ __attribute__((aligned(16))) u16 Bs[2][LBN * LLD];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    const int TM = (M + LBM - 1) / LBM, TN = (N + LBN - 1) / LBN, total = TM * TN;
    const int id = blockIdx.x, per = total / 8;
    const int t = id < 8 * per ? (id % 8) * per + id / 8 : id;
    const int gsz = GROUP_M * TN;
    const int first_m = (t / gsz) * GROUP_M;
    const int gm = min(TM - first_m, GROUP_M);
    const int tm = first_m + (t % gsz) % gm, tn = (t % gsz) / gm;
    const int m0 = tm * LBM, n0 = tn * LBN;
    const int KQ = K >> 5, NT = (N + 15) >> 4;

    // staging: 8 A and 8 B pieces of 16 bytes per thread and k-tile
    const u16* ag[8];
    const u16* bg[8];
    int sa[8], sb[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int c = tid + 256 * j;
        const int row = c >> 3, ch = c & 7;
        ag[j] = x + (size_t)min(m0 + row, M - 1) * K + ch * 8;
        sa[j] = lds_off(row, ch);
        if (WL == W_FRAG) {  // piece c of the 32 fragment blocks (16 n-tiles x 2 k-steps) of the tile
            const int blk = c >> 6, l = c & 63;
            const int ntl = blk >> 1, kql = blk & 1;
            bg[j] = w + ((size_t)min((n0 >> 4) + ntl, NT - 1) * KQ + kql) * 512 + l * 8;
            sb[j] = lds_off(16 * ntl + (l & 15), 4 * kql + (l >> 4));
        } else {
            bg[j] = w + (size_t)min(n0 + row, N - 1) * K + ch * 8;
            sb[j] = lds_off(row, ch);
        }
    }
    constexpr int BSTEP = WL == W_FRAG ? 1024 : LBK;  // elements per k-tile along a B piece's stream
    const int nk = K / LBK;

    u16x8 ra0[8], rb0[8], ra1[8], rb1[8];
    auto gload = [&](u16x8* ra, u16x8* rb, int kt) {
        const int k = min(kt, nk - 1);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            ra[j] = *reinterpret_cast<const u16x8*>(ag[j] + (size_t)k * LBK);
            rb[j] = *reinterpret_cast<const u16x8*>(bg[j] + (size_t)k * BSTEP);
        }
    };
    auto lstore = [&](const u16x8* ra, const u16x8* rb, int buf) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            *reinterpret_cast<u16x8*>(&As[buf][sa[j]]) = ra[j];
            *reinterpret_cast<u16x8*>(&Bs[buf][sb[j]]) = rb[j];
        }
    };

    f32x16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    const int fr = lane & 31, fh = lane >> 5;
    int aoff[4], boff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        aoff[i] = wm * 128 + i * 32 + fr;
        boff[i] = wn * 128 + i * 32 + fr;
    }
    auto rdfrag = [&](int buf, int s, bf16x8* a, bf16x8* b) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            a[i] = *reinterpret_cast<const bf16x8*>(&As[buf][lds_off(aoff[i], 2 * s + fh)]);
            b[i] = *reinterpret_cast<const bf16x8*>(&Bs[buf][lds_off(boff[i], 2 * s + fh)]);
        }
    };
    auto mma = [&](const bf16x8* a, const bf16x8* b) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = mfma32(a[i], b[j], acc[i][j]);
    };
    // one k-tile on LDS buffer `buf`, loading tile kt_ld into (ra_ld, rb_ld) and storing (ra_st, rb_st)
    // into the other buffer
    auto tile = [&](int buf, u16x8* ra_ld, u16x8* rb_ld, const u16x8* ra_st, const u16x8* rb_st, int kt_ld) {
        bf16x8 a0[4], b0[4], a1[4], b1[4];
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
        // 8 fragment reads up front; then per k-16 sub-step 16 MFMAs, each of the first 8 followed by a
        // fragment read (sub-steps 0-2), the last 8 by two global loads (0-1) or an LDS store (2); in
        // sub-step 3 the first 8 by an LDS store
        __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
        for (int ss = 0; ss < 4; ++ss)
            for (int m = 0; m < 16; ++m) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                if (ss < 3 && m < 8)
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                else if (ss < 2)
                    __builtin_amdgcn_sched_group_barrier(0x020, 2, 0);
                else if ((ss == 2 && m >= 8) || (ss == 3 && m < 8))
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

    // C layout of 32x32 MFMA: lane l, element e -> row 8*(e/4) + 4*(l/32) + e%4, column l % 32.
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int col = n0 + wn * 128 + j * 32 + (lane & 31);
            if (col >= N) continue;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = m0 + wm * 128 + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                if (row < M) store_out<OUT>(y, (size_t)row * N + col, acc[i][j][e]);
            }
        }
}

template <int NTS, int MT, int NW, int WL, int XL>
hipError_t gemv(const void* x, const void* w, int M, int N, int K, void* y, int out_kind, hipStream_t stream) {
    constexpr int PD = 4;
    const dim3 grid((N + NTS * 16 - 1) / (NTS * 16));
    const dim3 block(NW * 64);
    if (out_kind == OUT_F32)
        hipLaunchKernelGGL((gemv_kernel<NTS, MT, NW, PD, OUT_F32, WL, XL>), grid, block, 0, stream, (const u16*)x,
                           (const u16*)w, M, N, K, y);
    else
        hipLaunchKernelGGL((gemv_kernel<NTS, MT, NW, PD, OUT_BF16, WL, XL>), grid, block, 0, stream, (const u16*)x,
                           (const u16*)w, M, N, K, y);
    return hipGetLastError();
}

// Shape choice: enough workgroups to spread over the 256 CUs (NTS = rows / 16 per workgroup) and
// enough waves per workgroup to keep >= 8 k-steps of 32 per wave.  Measured on the 9B shape at M = 64:
// in_proj (N 12352, K 4096) NTS 4 / NW 4, out_proj (N 4096, K 4096) NTS 1 / NW 8.
template <int MT, int WL, int XL>
hipError_t gemv_mt(const void* x, const void* w, int M, int N, int K, void* y, int out_kind, hipStream_t stream) {
    const int NT = (N + 15) / 16, KQ = K / 32;
    if (NT >= 4 * 160) {
        if (KQ >= 64) return gemv<4, MT, 4, WL, XL>(x, w, M, N, K, y, out_kind, stream);
        return gemv<4, MT, 2, WL, XL>(x, w, M, N, K, y, out_kind, stream);
    }
    if (NT >= 2 * 160) {
        if (KQ >= 64) return gemv<2, MT, 8, WL, XL>(x, w, M, N, K, y, out_kind, stream);
        return gemv<2, MT, 4, WL, XL>(x, w, M, N, K, y, out_kind, stream);
    }
    if (KQ >= 64) return gemv<1, MT, 8, WL, XL>(x, w, M, N, K, y, out_kind, stream);
    return gemv<1, MT, 4, WL, XL>(x, w, M, N, K, y, out_kind, stream);
}

template <int WL, int XL>
hipError_t gemv_m(const void* x, const void* w, int M, int N, int K, void* y, int out_kind, hipStream_t stream) {
    if (M <= 16) return gemv_mt<1, WL, XL>(x, w, M, N, K, y, out_kind, stream);
    if (M <= 32) return gemv_mt<2, WL, XL>(x, w, M, N, K, y, out_kind, stream);
    if (M <= 48) return gemv_mt<3, WL, XL>(x, w, M, N, K, y, out_kind, stream);
    return gemv_mt<4, WL, XL>(x, w, M, N, K, y, out_kind, stream);
}

template <int WL>
hipError_t linear_wl(const void* x, int xlayout, const void* w, int M, int N, int K, void* y, int out_kind,
                     hipStream_t stream) {
    if (M <= 64) {
        if (xlayout == W_FRAG) return gemv_m<WL, W_FRAG>(x, w, M, N, K, y, out_kind, stream);
        return gemv_m<WL, W_ROW>(x, w, M, N, K, y, out_kind, stream);
    }
    if (xlayout != W_ROW) return hipErrorInvalidValue;  // the GEMM reads row-major activations
    if ((size_t)M * N >= (size_t)256 * 256 * 256) {  // >= one round of 256 x 256 tiles over the CUs
        const dim3 grid(((M + LBM - 1) / LBM) * ((N + LBN - 1) / LBN));
        if (out_kind == OUT_F32)
            hipLaunchKernelGGL((gemm256_kernel<OUT_F32, WL>), grid, dim3(256), 0, stream, (const u16*)x,
                               (const u16*)w, M, N, K, y);
        else
            hipLaunchKernelGGL((gemm256_kernel<OUT_BF16, WL>), grid, dim3(256), 0, stream, (const u16*)x,
                               (const u16*)w, M, N, K, y);
        return hipGetLastError();
    }
    const dim3 grid(((M + TBM - 1) / TBM) * ((N + TBN - 1) / TBN));
    if (out_kind == OUT_F32)
        hipLaunchKernelGGL((gemm_kernel<OUT_F32, WL>), grid, dim3(256), 0, stream, (const u16*)x, (const u16*)w, M,
                           N, K, y);
    else
        hipLaunchKernelGGL((gemm_kernel<OUT_BF16, WL>), grid, dim3(256), 0, stream, (const u16*)x, (const u16*)w,
                           M, N, K, y);
    return hipGetLastError();
}

}  // namespace

size_t frag_elems(int N, int K) { return (size_t)((N + 15) / 16) * 16 * K; }

hipError_t launch_frag_tile(const void* w, int N, int K, void* wf, hipStream_t stream) {
    const size_t pieces = frag_elems(N, K) / 8;
    hipLaunchKernelGGL(frag_tile_kernel, dim3((unsigned)((pieces + 255) / 256)), dim3(256), 0, stream, (const u16*)w,
                       N, K, (u16*)wf);
    return hipGetLastError();
}

namespace {

template <int MT>
hipError_t in_proj_decode_mt(const void* x, const void* w, int M, int N1, int N2, int K, float* P, int ldp,
                             float* Pab, int ab_splits, hipStream_t stream) {
    constexpr int PD = 4, NW = 4;
    const int NT1 = N1 >> 4, NT2 = (N2 + 15) >> 4;
    // tiles per workgroup: the smallest that keeps the main workgroups within one per CU
    const int nts = NT1 <= 256 ? 1 : (NT1 <= 512 ? 2 : (NT1 <= 768 ? 3 : 4));
    if (NT1 % nts) return hipErrorInvalidValue;
    const int G = NT1 / nts;
    const dim3 grid(G + NT2 * ab_splits), block(NW * 64);
    const u16 *xs = (const u16*)x, *ws = (const u16*)w;
    switch (nts) {
        case 1: hipLaunchKernelGGL((in_proj_decode_kernel<1, MT, NW, PD>), grid, block, 0, stream, xs, ws, M, N1, N2, K, G, ab_splits, P, ldp, Pab); break;
        case 2: hipLaunchKernelGGL((in_proj_decode_kernel<2, MT, NW, PD>), grid, block, 0, stream, xs, ws, M, N1, N2, K, G, ab_splits, P, ldp, Pab); break;
        case 3: hipLaunchKernelGGL((in_proj_decode_kernel<3, MT, NW, PD>), grid, block, 0, stream, xs, ws, M, N1, N2, K, G, ab_splits, P, ldp, Pab); break;
        default: hipLaunchKernelGGL((in_proj_decode_kernel<4, MT, NW, PD>), grid, block, 0, stream, xs, ws, M, N1, N2, K, G, ab_splits, P, ldp, Pab); break;
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_in_proj_decode(const void* x_frag, const void* w_frag, int M, int N1, int N2, int K, float* P,
                                 int ldp, float* Pab, int ab_splits, hipStream_t stream) {
    if (M <= 0) return hipSuccess;
    if (M > 64 || N1 % 16 || ab_splits <= 0 || K % 32) return hipErrorInvalidValue;
    if (M <= 16) return in_proj_decode_mt<1>(x_frag, w_frag, M, N1, N2, K, P, ldp, Pab, ab_splits, stream);
    if (M <= 32) return in_proj_decode_mt<2>(x_frag, w_frag, M, N1, N2, K, P, ldp, Pab, ab_splits, stream);
    if (M <= 48) return in_proj_decode_mt<3>(x_frag, w_frag, M, N1, N2, K, P, ldp, Pab, ab_splits, stream);
    return in_proj_decode_mt<4>(x_frag, w_frag, M, N1, N2, K, P, ldp, Pab, ab_splits, stream);
}

hipError_t launch_linear(const void* x, int xlayout, const void* w, int wlayout, int M, int N, int K, void* y,
                         int out_kind, hipStream_t stream) {
    if (M <= 0 || N <= 0) return hipSuccess;
    if (wlayout == W_FRAG) return linear_wl<W_FRAG>(x, xlayout, w, M, N, K, y, out_kind, stream);
    return linear_wl<W_ROW>(x, xlayout, w, M, N, K, y, out_kind, stream);
}

}  // namespace gdn

// Shared device helpers and internal launcher declarations for the Gated DeltaNet HIP library.
// gfx950 (CDNA4) only: 64-wide wavefronts, bf16 MFMA, 160 KB LDS per CU.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gdn {

typedef __bf16 bf16;
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint16_t u16;
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint8_t u8;

constexpr int WAVE = 64;

__device__ __forceinline__ float bf2f(u16 b) { return __uint_as_float((uint32_t)b << 16); }

// fp32 -> bf16 bits, round to nearest even (NaN kept quiet).
__device__ __forceinline__ u16 f2bf(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u16)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (u16)(u >> 16);
}

__device__ __forceinline__ float warp_sum(float x) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, WAVE);
    return x;
}

// Sum over lanes that share (lane % width); width is a power of two <= 64.
template <int WIDTH>
__device__ __forceinline__ float lane_group_sum(float x) {
#pragma unroll
    for (int off = WIDTH; off < WAVE; off <<= 1) x += __shfl_xor(x, off, WAVE);
    return x;
}

// ---- MFMA (gfx950 bf16) -----------------------------------------------------------------------
// v_mfma_f32_16x16x32_bf16: lane l holds A[l % 16][8 (l / 16) + j] and B[8 (l / 16) + j][l % 16],
// j = 0..7; C element i of lane l is C[4 (l / 16) + i][l % 16].
__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
// v_mfma_f32_32x32x16_bf16: lane l holds A[l % 32][8 (l / 32) + j]; C element e of lane l is
// C[8 (e / 4) + 4 (l / 32) + e % 4][l % 32].
__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// fp32 operands on bf16 MFMA at ~fp32 accuracy: x = hi + lo with hi = bf16(x), lo = bf16(x - hi)
// (relative error ~2^-17), and a.b ~= a_hi.b_hi + a_hi.b_lo + a_lo.b_hi (the lo.lo term is below
// fp32 rounding).  The small terms are accumulated first.
struct Split8 {
    bf16x8 h, l;
};
__device__ __forceinline__ Split8 split8(const float* v) {
    Split8 s;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const __bf16 hi = (__bf16)v[j];
        s.h[j] = hi;
        s.l[j] = (__bf16)(v[j] - (float)hi);
    }
    return s;
}
__device__ __forceinline__ f32x4 mfma3(const Split8& a, const Split8& b, f32x4 c) {
    c = mfma16(a.l, b.h, c);
    c = mfma16(a.h, b.l, c);
    return mfma16(a.h, b.h, c);
}

// ---- FP8 (OCP E4M3: 1 sign, 4 exponent bits biased by 7, 3 mantissa bits; largest finite 448) --------
// Encoding of one value, round to nearest even, saturating to +-448 (the weight quantizer).
__host__ __device__ __forceinline__ uint32_t e4m3_code(float v) {
    union { float f; uint32_t u; } b{v};
    const uint32_t sign = (b.u >> 24) & 0x80u;
    const float a = fminf(fabsf(v), 448.0f);
    if (a < 0.015625f) return sign | (uint32_t)rintf(a * 512.0f);  // subnormal steps of 2^-9 (8 = 2^-6)
    b.f = a;
    const uint32_t u = b.u + 0x7ffffu + ((b.u >> 20) & 1u);         // keep 3 mantissa bits, ties to even
    return sign | (((u >> 23) - 120u) << 3) | ((u >> 20) & 7u);
}

// 16 E4M3 values (bytes in k order) -> 2 x 8 bf16, exact (every E4M3 value is a bf16 value).
__device__ __forceinline__ void e4m3x16_to_bf16(const u32x4 q, bf16x8& lo, bf16x8& hi) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    bf16x2 p[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        p[2 * i] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q[i], 1.0f, false);     // bytes 0, 1
        p[2 * i + 1] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q[i], 1.0f, true);  // bytes 2, 3
    }
    lo = bf16x8{p[0][0], p[0][1], p[1][0], p[1][1], p[2][0], p[2][1], p[3][0], p[3][1]};
    hi = bf16x8{p[4][0], p[4][1], p[5][0], p[5][1], p[6][0], p[6][1], p[7][0], p[7][1]};
}

// ---- MXFP4 (OCP Microscaling: E2M1 values 0, 0.5, 1, 1.5, 2, 3, 4, 6 with one E8M0 scale per 32) -------
// E2M1 code of one value already divided by its block scale: nearest, ties to the even mantissa,
// saturating to +-6 (the decision thresholds of that rounding on the E2M1 grid).
__host__ __device__ __forceinline__ uint32_t e2m1_code(float v) {
    const float a = fabsf(v);
    const uint32_t c = a <= 0.25f ? 0u : a < 0.75f ? 1u : a <= 1.25f ? 2u : a < 1.75f ? 3u
                     : a <= 2.5f ? 4u : a < 3.5f ? 5u : a <= 5.0f ? 6u : 7u;
    return (signbit(v) ? 8u : 0u) | c;
}
// E8M0 exponent byte of the block scale 2^(floor(log2 amax) - EMAX), clamped to [-127, 127]; 0 for amax 0.
// EMAX is the exponent of the element format's largest power of two: 2 for E2M1, 0 for MXINT8.
template <int EMAX = 2>
__host__ __device__ __forceinline__ uint32_t mx_scale_code(float amax) {
    if (!(amax > 0.f)) return 0u;
    union { float f; uint32_t u; } b{amax};
    int e = (int)((b.u >> 23) & 0xffu) - 127;  // floor(log2 amax) for a normal amax
    if (((b.u >> 23) & 0xffu) == 0u) e = -127;  // subnormal amax: below 2^-126, the clamp applies
    int x = e - EMAX;
    x = x < -127 ? -127 : (x > 127 ? 127 : x);
    return (uint32_t)(x + 127);
}

// The scale of an E8M0 byte as a float (2^-127 for code 0, a subnormal).
__device__ __forceinline__ float e8m0_value(uint32_t e) { return __uint_as_float(e ? e << 23 : 0x00400000u); }
// 8 E2M1 codes (4 bytes, two per byte, low nibble first, in k order) times `scale` -> 8 bf16, exact for
// scales of at least 2^-126 (every such product is a bf16 value).
__device__ __forceinline__ bf16x8 e2m1x8_to_bf16(uint32_t q, float scale) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    const bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, scale, 0);
    const bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, scale, 1);
    const bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, scale, 2);
    const bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, scale, 3);
    return bf16x8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

// ---- MXINT8 (OCP Microscaling: two's-complement int8 elements worth code * 2^-6, one E8M0 scale per 32) ---
// The counterpart of bfloat8_b (7 significant bits under an exponent shared by a block).  Code of one value
// already divided by its block scale: 64 v rounded to nearest, ties to even, saturated to [-128, 127].
__host__ __device__ __forceinline__ int32_t i8_code(float v) {
    const float c = rintf(v * 64.0f);
    return (int32_t)(c < -128.f ? -128.f : (c > 127.f ? 127.f : c));
}
// The weight of a code step under scale byte e, 2^(e - 127) * 2^-6 = 2^(e - 133), as a float (a subnormal
// for e < 7).
__device__ __forceinline__ float i8_step(uint32_t e) {
    return __uint_as_float(e >= 7u ? (e - 6u) << 23 : 1u << (e + 16u));
}
// 16 MXINT8 codes (bytes in k order: the 8 of k-step 0, then the 8 of k-step 1) -> 2 x 8 bf16, k-step h
// times its step s_h.  Byte b + 128 goes through v_cvt_f32_ubyte and one fma: (b + 128) s - 128 s = b s,
// exact (b s is a bf16 value for steps of at least 2^-126: scale bytes >= 7).
__device__ __forceinline__ void i8x16_to_bf16(const u32x4 q, float s0, float s1, bf16x8& lo, bf16x8& hi) {
    float v[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t u = q[i] ^ 0x80808080u;
        const float s = i < 2 ? s0 : s1, o = -128.0f * s;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[4 * i + j] = fmaf((float)((u >> (8 * j)) & 0xffu), s, o);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) lo[j] = (__bf16)v[j], hi[j] = (__bf16)v[8 + j];
}

// Workgroup barrier for LDS traffic only: unlike __syncthreads() it does not wait for outstanding
// global loads, so loads issued for the next step stay in flight across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// The reciprocals use the hardware v_rcp_f32 (1 ulp) instead of an IEEE division sequence.
__device__ __forceinline__ float sigmoidf_(float x) { return __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }
__device__ __forceinline__ float siluf_(float x) { return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }
// torch.nn.functional.softplus with beta = 1, threshold = 20
__device__ __forceinline__ float softplusf_(float x) { return x > 20.0f ? x : log1pf(__expf(x)); }

}  // namespace gdn

// ------------------------------------------------------------------------------------------------
// Internal launchers (each returns a hipError_t of the launch).  Pointers are device pointers.
// ------------------------------------------------------------------------------------------------
namespace gdn {

// OUT_F32_T: fp32, element (m, n) stored at n * ldy + m (the transposed GEMV below)
enum OutKind { OUT_F32 = 0, OUT_BF16 = 1, OUT_F32_T = 2 };
// Weight layouts: W_ROW = row-major bf16 [N, K]; W_FRAG = bf16 MFMA-fragment blocks; W_F8 = E4M3 fragment
// blocks with one fp32 scale per row; W_F4 = MXFP4 fragment blocks with one E8M0 scale per row and 32
// columns (see gdn_linear.hip).
// W_I8 = MXINT8 codes in the W_F8 block order with one E8M0 scale per row and 32 columns in the W_F4 scale order
// (see gdn_linear.hip).
enum WLayout { W_ROW = 0, W_FRAG = 1, W_F8 = 2, W_F4 = 3, W_I8 = 4 };

// y[M, N] (row stride ldy) = x[M, K] . w[N, K]^T ; bf16 activations, fp32 accumulation; K % 128 == 0.
// w in layout `wlayout` (W_F8: w = E4M3 codes, row n scaled by w_scale[n]; W_F4: w = E2M1 codes, w_scale
// the E8M0 scale codes in f4_scale_offset order, passed through this pointer); x in `xlayout` (W_FRAG
// activations only for M <= 64).
hipError_t launch_linear(const void* x, int xlayout, const void* w, int wlayout, const float* w_scale, int M, int N,
                         int K, void* y, int ldy, int out_kind, hipStream_t stream);
// y[n * ldy + m] = sum_k w[m][k] x[n][k] for a few weight rows (M <= 64, w in W_FRAG layout) against many
// row-major activation rows x [N, K] (K % 32 == 0): the GEMV with the roles swapped, so that a skinny
// projection of a long prefill (the a | b rows) streams the activations once over every CU.
hipError_t launch_linear_rows_t(const void* x, const void* w, int M, int N, int K, float* y, int ldy,
                                hipStream_t stream);
// Decode in_proj (M <= 64; activations in W_FRAG layout, or row-major W_ROW for M <= 16): rows [0, N1) of w
// (W_FRAG, or W_F8 / W_F4 with w_scale) into P (fp32, row stride ldp) with the workgroups balanced over the CUs;
// the N2 rows of w2 (W_FRAG) as ab_splits partial sums over k ranges into Pab [ab_splits][M][N2] (the
// consumer adds the slices).  N1 % 16 == 0.
hipError_t launch_in_proj_decode(const void* x, int xlayout, const void* w, int wlayout, const float* w_scale,
                                 const void* w2, int M, int N1, int N2, int K, float* P, int ldp, float* Pab,
                                 int ab_splits, hipStream_t stream);
// Whether launch_in_proj_decode takes N1 rows of K columns (its workgroups tile the rows evenly).
bool in_proj_decode_supported(int N1, int K);
// Elements of an [N, K] matrix in W_FRAG layout (rows padded to a multiple of 16); also the bytes of the
// same matrix in W_F8 layout.
size_t frag_elems(int N, int K);
// Quantize a row-major bf16 [N, K] matrix to E4M3 with per-row scale absmax / 448 (1 for a zero row):
// codes in W_F8 layout (to_frag != 0; rows padded to 16 with zeros, K % 64 == 0) or row-major [N, K].
hipError_t launch_quantize_e4m3(const void* w, int N, int K, u8* q, float* scale, int to_frag, hipStream_t stream);
// Byte offset of (row n, column k) of an [N, K] matrix in W_F8 layout: blocks of 16 rows x 64 columns
// (1 KB), lane l = 16 g + r of block holding the 16 bytes W[16 nt + r][64 kp + 32 h + 8 g + j] at
// 16 l + 8 h + j -- two consecutive MFMA A operands per 16-byte load.
__host__ __device__ __forceinline__ size_t f8_offset(int n, int k, int K) {
    return ((size_t)(n >> 4) * (K >> 6) + (k >> 6)) * 1024 + ((((k >> 3) & 3) << 4) + (n & 15)) * 16 +
           ((k >> 5) & 1) * 8 + (k & 7);
}
// MXFP4 weights: codes in W_F4 layout (to_frag != 0; rows padded to 16 with zero codes and scale code 0,
// K % 128 == 0) or row-major [N, K / 2] bytes (low nibble = even column), with their E8M0 scale codes in
// the matching order (f4_scale_offset, or row-major [N, K / 32]).
hipError_t launch_quantize_mxfp4(const void* w, int N, int K, u8* q, u8* scale, int to_frag, hipStream_t stream);
// MXINT8 weights: int8 codes in W_I8 layout (to_frag != 0: the W_F8 block order, rows padded to 16 with zero codes
// and scale code 0, K % 128 == 0) or row-major [N, K], with their E8M0 scale codes in f4_scale_offset order (or
// row-major [N, K / 32]).
hipError_t launch_quantize_mxint8(const void* w, int N, int K, u8* q, u8* scale, int to_frag, hipStream_t stream);
// W_F4 layout: blocks of 16 rows x 128 columns (1 KB), lane l = 16 g + r of block holding the 32 codes
// W[16 nt + r][128 kb + 32 h + 8 g + j] (h, j < 4, 8) in its 16 bytes at byte 4 h + j / 2, nibble j % 2 --
// four consecutive MFMA A operands per 16-byte load.  Byte offset of (row n, column k):
__host__ __device__ __forceinline__ size_t f4_offset(int n, int k, int K) {
    return ((size_t)(n >> 4) * (K >> 7) + (k >> 7)) * 1024 + ((((k >> 3) & 3) << 4) + (n & 15)) * 16 +
           ((k >> 5) & 3) * 4 + ((k & 7) >> 1);
}
// Scale codes of W_F4: [N / 16][K / 128][16 rows][4 k-steps] bytes, so the lane of row r reads the scales of
// its four k-steps as one 32-bit word.  Byte offset of the scale of (row n, 32-column block kq):
__host__ __device__ __forceinline__ size_t f4_scale_offset(int n, int kq, int K) {
    return (((size_t)(n >> 4) * (K >> 7) + (kq >> 2)) * 16 + (n & 15)) * 4 + (kq & 3);
}
// Convert a row-major device matrix [N, K] into W_FRAG layout (frag_elems(N, K) elements).
hipError_t launch_frag_tile(const void* w, int N, int K, void* wf, hipStream_t stream);
// Element offset of (row n, column k) of an [N, K] matrix in W_FRAG layout.
__host__ __device__ __forceinline__ size_t frag_offset(int n, int k, int K) {
    return ((size_t)(n >> 4) * (K >> 5) + (k >> 5)) * 512 + ((((k >> 3) & 3) << 4) + (n & 15)) * 8 + (k & 7);
}

// Conv history ring of a state slot, one per k-head group (k-head kh with its R = nv / nk v-heads):
// [4][2 dk + R dv] fp32 entries of the pre-conv inputs of the group's channels -- q and k of kh, then v of the
// v-heads R kh .. R kh + R - 1.  The input of absolute token time tau sits at entry tau % 4; pos = (tokens seen)
// % 4 is kept per (slot, v-head) in conv_pos [slots, nv] (every v-head's copy of a slot is equal).  The
// window of the next token, time order j = 0 (oldest) .. 2 (newest), is entry (pos + 1 + j) % 4, and the
// launch's input t (0-based) goes to entry (pos + t) % 4; a launch writes only its last min(T, 3) inputs,
// one entry per token, and entries that stay in the window do not move (the roll of layer_reader.cpp:184-197
// without the copy).  With four entries a single-token launch writes the one entry no window reads, so the
// v-heads of a group may run in separate workgroups that all read the group's q and k history while one of
// them writes it; every workgroup advances only its own v-head's position.
constexpr int CONV_RING = 4;
__host__ __device__ __forceinline__ int conv_group_width(int dk, int dv, int R) { return 2 * dk + R * dv; }
__host__ __device__ __forceinline__ int ring_index(int pos, int j) { return (pos + 1 + j) & 3; }
__host__ __device__ __forceinline__ int ring_put(int pos, int t) { return (pos + t) & 3; }
// Column in the fused projection row (q | k | v | z | a | b) of channel c of group kh (Kd = nk dk).
__host__ __device__ __forceinline__ int group_col(int c, int kh, int dk, int dv, int R, int Kd) {
    return c < dk ? kh * dk + c : (c < 2 * dk ? Kd + kh * dk + (c - dk) : 2 * Kd + kh * R * dv + (c - 2 * dk));
}

struct MixerArgs {
    const float* P;         // [M, NP] fused projection rows (q | k | v | z | a | b)
    int NP;                 // row stride of P
    int B, T;               // launch = B sequences x T tokens, rows m = b * T + t
    const int* slot_ids;    // [B] device, or nullptr for identity
    int max_slots;          // slots of the state buffers; a sequence whose slot id is outside is skipped
    int nk, nv;             // heads
    const float4* conv_w;   // [conv_dim] taps (w0, w1, w2, w3) per channel
    const float* neg_A;     // [nv]  -exp(A_log)
    const float* dt_bias;   // [nv]
    const float* norm_w;    // [dv]
    float eps;              // RMSNorm eps
    float* rec_state;       // [slots, nv, dk, dv]
    float* conv_state;      // [slots, nk, 4, 2 dk + R dv] conv history rings
    int* conv_pos;          // [slots, nv] ring positions
    u16* y;                 // [M, nv * dv] bf16 gated RMSNorm output
    int y_frag;             // 1: y in W_FRAG layout (rows padded to 16; M <= 64), 0: row-major
    float* o_tap;           // optional [M, nv * dv] recurrence output (nullptr: not written)
    // split heads (single-token launches of at most 64 sequence-heads, 128-wide heads): when set, each
    // v-head runs as kMixerSplit workgroups of dv / kMixerSplit state columns that write the recurrence
    // output to o_tap and their partial sums of its squares to ss_part [M, nv, kMixerSplit] instead of y,
    // and leave conv_pos to launch_out_proj_gnorm (see there)
    float* ss_part;
    // optional: a | b as ab_splits partial sums, slice s row m at ab[s * ab_stride + m * 2 nv] (then
    // the a | b columns of P are not read)
    const float* ab;
    int ab_splits;
    size_t ab_stride;
};
// Fused mixer of a decode-sized launch: single-token launches one workgroup of 256 threads per (sequence,
// v-head); longer ones one workgroup of 256 R threads per (sequence, k-head group), R = nv / nk <= 4.
hipError_t launch_mixer(const MixerArgs& a, int dk, int dv, hipStream_t stream);
constexpr int kMixerSplit = 4;  // workgroups per v-head of a split-head launch

// The out_proj of a split-head mixer launch (MixerArgs::ss_part): the gated RMSNorm of its rows, then the
// projection (bf16, E4M3, MXFP4 or MXINT8 weights); it also advances the ring positions of the launch's
// sequences by the one token, which the split mixer leaves to it.
struct GnormArgs {
    const float* o;        // [M, K] recurrence output (K = nv dv)
    const float* ss;       // [M, nv, kMixerSplit] partial sums of squares of o per head and column slice
    const float* z;        // gate rows: row m at z + m ldz
    int ldz;
    const float* norm_w;   // [dv]
    float eps;
    int nv, dv;
    const void* w;         // [N, K]: bf16 W_FRAG, or E4M3 / MXFP4 / MXINT8 fragments (the layout argument)
    const float* scale;    // the weights' scales (W_F8 per row; W_F4, W_I8 the E8M0 codes); nullptr for bf16
    int M, N, K;
    void* y;               // [M, N] row-major, bf16 or fp32 by the out kind
    int ldy;
    int* conv_pos;         // [slots, nv]
    const int* slot_ids;   // [M] (nullptr: identity)
    int max_slots;
};
constexpr int kGnormMaxM = 4, kGnormMaxK = 4096;
hipError_t launch_out_proj_gnorm(const GnormArgs& a, int wlayout, int out_kind, hipStream_t stream);

struct FrontArgs {
    const float* P;
    int NP;
    int B, T;
    const int* slot_ids;
    int max_slots;            // sequences with a slot id outside [0, max_slots) are skipped
    int nk, nv, dk, dv;
    const float4* conv_w;
    const float* neg_A;
    const float* dt_bias;
    const float* conv_state;  // history rings (read only here)
    const int* conv_pos;      // ring positions
    float* qn;                // [M, nk, dk]  l2norm(q) * dk^-0.5
    float* kn;                // [M, nk, dk]  l2norm(k)
    float* v;                 // [M, nv, dv]
    float* g;                 // [M, nv]
    float* beta;              // [M, nv]
};
hipError_t launch_conv_front(const FrontArgs& a, hipStream_t stream);
// Roll each sequence's conv history rings forward over the T inputs of this launch.
hipError_t launch_conv_commit(const float* P, int NP, int B, int T, const int* slot_ids, int max_slots, int nk,
                              int nv, int dk, int dv, float* conv_state, int* conv_pos, hipStream_t stream);

// Recurrence over T tokens for B sequences from pre-normalised q/k (qn already scaled).
struct DeltaArgs {
    const float* q;        // [B*T, Hk, dk]
    const float* k;        // [B*T, Hk, dk]
    const float* v;        // [B*T, Hv, dv]
    const float* g;        // [B*T, Hv]
    const float* beta;     // [B*T, Hv]
    int B, T, Hk, Hv;
    const int* slot_ids;   // state slot of sequence b (nullptr: b)
    int max_slots;         // slots of `state`; a sequence whose slot id is outside [0, max_slots) is skipped
    float* state;          // [slots, Hv, dk, dv]
    float* o;              // [B*T, Hv, dv]
    int normalize;         // 1: apply l2norm to q/k in the kernel
    float scale;           // q scale applied in the kernel (1 when q is pre-scaled)
};
hipError_t launch_delta_seq(const DeltaArgs& a, int dk, int dv, hipStream_t stream);
// Chunk-64 form for long prefills (dk == dv == 128); `workspace` of delta_chunked_workspace() bytes.
hipError_t launch_delta_chunked(const DeltaArgs& a, int dk, int dv, void* workspace, size_t ws_bytes,
                                hipStream_t stream);
size_t delta_chunked_workspace(int B, int T, int Hv, int dk, int dv);
// The same with the front end fused into the chunk preparation: q, k, v, g, beta of each chunk are computed
// from the projection rows f.P (conv history f.conv_state, then rolled forward in conv_state), so f.qn ..
// f.beta and r.q .. r.beta are not used; r carries B, T, heads, slots, the state and o.
hipError_t launch_front_chunked(const FrontArgs& f, float* conv_state, int* conv_pos, const DeltaArgs& r,
                                void* workspace, size_t ws_bytes, hipStream_t stream);
bool delta_chunked_supported(int dk, int dv);

// y = o * rsqrt(mean(o^2) + eps) * w * silu(z), per head of dv; y bf16.
// Decoder RMSNorm of M rows of H bf16 values: y = x rsqrt(mean(x^2) + eps) (1 + w), w fp32 [H] or NULL
// (= 0).  H % 8 == 0, H <= 8192.  In place (y == x) is allowed.
hipError_t launch_rmsnorm_rows(const u16* x, int M, int H, const float* w, float eps, u16* y, hipStream_t stream);
hipError_t launch_gated_rmsnorm(const float* o, int M, int nv, int dv, const float* z, int z_stride,
                                const float* w, float eps, u16* y, hipStream_t stream);

// State import / export / zero of n slots (ids outside [0, max_slots) are skipped): recurrent state
// [n, nv, dk, dv]; conv history in the reference's time order [n, conv_dim, 3] (entry 2 newest), translated
// from and to the rings (import and zero set the ring positions to 0).
hipError_t launch_state_export(const float* rec_state, const float* conv_state, const int* conv_pos, const int* slots,
                               int n, int max_slots, int nk, int nv, int dk, int dv, float* rec_out, float* conv_out,
                               hipStream_t stream);
hipError_t launch_state_import(float* rec_state, float* conv_state, int* conv_pos, const int* slots, int n,
                               int max_slots, int nk, int nv, int dk, int dv, const float* rec_in,
                               const float* conv_in, hipStream_t stream);
hipError_t launch_state_zero(float* rec_state, float* conv_state, int* conv_pos, const int* slots, int n,
                             int max_slots, int nk, int nv, int dk, int dv, hipStream_t stream);

}  // namespace gdn

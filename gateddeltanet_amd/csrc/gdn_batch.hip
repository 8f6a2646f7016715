// gdn_batch.hip -- multi-stream decode: up to 64 independent token streams,
// each with its own recurrent and conv state, advanced one token per stream
// per step.  The reference decodes a single stream (README.md:75-77); this
// path keeps its per-stream arithmetic and moves the projections onto the
// matrix cores.
//
// Arithmetic.  Every operator outside the projections is the BF16W_FP32S
// arithmetic of the batch-1 engine (the same device functions): embedding
// import, residual adds and RMSNorms in chunk order, the tiny a/b rows in
// FP32 products, conv + SiLU with the tail shift, beta/decay, the recurrence
// on an FP32 state, the output norm * gate, SwiGLU, FP32 logits and the
// strict-'>' argmax.  The projections take the same BF16 operands (weights
// and activations at their BF16 rounding points, subnormals flushed) but form
// exact products and accumulate them in FP32 on v_mfma_f32_16x16x32_bf16, in
// the matrix cores' order instead of the reference's tree16 + four banks.
// Results therefore agree with the batch-1 engine to rounding, not bit for
// bit; outputs are rounded to BF16 at the same points.
//
// Layout.  A projection W [N][K] is stored as MFMA A-operand tiles (16 rows x
// 32 columns, gdn_tile_bf16; gate/up in k_bgu's 44-row blocks, tile_gu).  The activations of all streams enter as the B
// operand: X [64 streams][K] BF16 in tiles of 32 columns x 16 streams, lane l
// holding stream l % 16 and columns 8 (l / 16) .. + 7.  Stream s of a GEMM
// output is column s of D = W X^T, so streams never mix.
//
// Per layer (8 launches):
//   k_bgemm<QKVG>  q,k,v,g rows; epilogue: BF16 rounding, conv + SiLU with
//                  each stream's tails, gate and sigmoid(gate)
//   k_brecur       the recurrence per (head, stream, 128 columns), state in registers
//   k_bonorm       per (head, stream) output RMSNorm * gate -> X
//   k_bgemm<RAW>   o_proj in 4 K splits -> split sums
//   k_bnorm        h = R(h + R(y)), MLP RMSNorm -> X
//   k_bgu          gate/up, 22 channels per workgroup, SwiGLU -> X (K = 5632)
//   k_bgemm<RAW>   down in 4 K splits -> split sums
//   k_bnorm        h = R(h + R(y)), next attention RMSNorm (or the final norm)
//                  -> X; with the next layer's a/b rows and beta/decay it runs
//                  four workgroups per stream, two heads' rows each
// plus the embedding norm before layer 0, the LM head with a per-workgroup
// argmax, and the per-stream argmax merge.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <vector>

#include "gdn_amd.h"
#include "gdn_device.h"
#include "gdn_internal.h"

namespace gdn {
namespace bt {

constexpr int kMaxB = GDN_MAX_STREAMS;  // streams = the 64 B-operand columns
static_assert(kMaxB == 64, "four 16-stream groups per MFMA B operand");
constexpr int kRecCols = 128;  // state columns per multi-stream recurrence workgroup
constexpr int kSplitO = 4;              // K splits of o_proj (16 k tiles each)
constexpr int kSplitDown = 4;           // K splits of the down projection (44 k tiles each)
constexpr int kRtO = 2;                 // 16-row tiles per o_proj workgroup
constexpr int kRtDown = 2;              // 16-row tiles per down workgroup
constexpr int kKtH = kH / 32;           // k tiles of a K = 2048 projection
constexpr int kKtI = kI / 32;           // k tiles of the down projection
constexpr size_t kLayerState = (size_t)kNH * kHD * kHD;  // floats per (layer, stream)
constexpr size_t kStreamTails = (size_t)3 * 3 * kH;      // floats per (layer, stream)

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

enum { EPI_RAW = 0, EPI_STORE = 1, EPI_QKVG = 2, EPI_LM = 4 };

// BF16 bits of a value already at a BF16 rounding point, subnormals flushed
// to a signed zero (the reference's products treat them as zero).
__device__ __forceinline__ uint32_t bf16_daz_bits(float v) {
    const uint32_t b = f2u(v);
    return ((b & 0x7f800000u) == 0u) ? ((b >> 16) & 0x8000u) : (b >> 16);
}

// Offset (BF16 elements) of (stream or token m, column k) in an X tile
// buffer of K columns: blocks of 64 streams (a step has one; a prefill
// segment one per 64 tokens), each [k tile][16-stream group][64 lanes][8].
__device__ __forceinline__ size_t xt_index(int m, int k, int K = kH) {
    const int kt = k >> 5, kk = k & 31, mm = m & 63;
    return (size_t)(m >> 6) * 64 * K +
           (size_t)((((kt * 4 + (mm >> 4)) * 64 + ((kk >> 3) << 4) + (mm & 15)) << 3) + (kk & 7));
}

// Eight consecutive columns k..k+7 (k % 8 == 0) of stream m in a K = kH X
// tile buffer, one 16-byte store.
__device__ __forceinline__ void store_x8(uint16_t *x, int m, int k, const float *v) {
    u32x4 w;
    w.x = bf16_daz_bits(v[0]) | (bf16_daz_bits(v[1]) << 16);
    w.y = bf16_daz_bits(v[2]) | (bf16_daz_bits(v[3]) << 16);
    w.z = bf16_daz_bits(v[4]) | (bf16_daz_bits(v[5]) << 16);
    w.w = bf16_daz_bits(v[6]) | (bf16_daz_bits(v[7]) << 16);
    *reinterpret_cast<u32x4 *>(x + xt_index(m, k)) = w;
}

// ------------------------------------------------------------ the GEMM

struct BEpi {
    int n_streams;
    int n_rows;          // N: row stride of y / logits
    float *y;            // EPI_RAW / EPI_STORE: [64][N]
    float *qkv;          // EPI_QKVG: [64][3][kH] after conv + SiLU
    float *gate;         // [64][kH] R(g)
    float *sgate;        // [64][kH] sigmoid(R(g))
    uint16_t *tails;     // this layer's [n_streams][3][3][kH], BF16 bits (the values are BF16)
    const float *conv_w; // [3][kH][4]
    float *logits;       // EPI_LM: [64][N]
    float *part_val;     // [gridDim.x][64]
    int *part_idx;
};

// D[rows][64 streams] = W[rows][K] X^T for 16 * RT rows per workgroup and
// KT / S k tiles (split S of the K range: grid (N / (16 RT), S)).  The NW
// waves split the workgroup's k tiles (wave w takes tiles w, w + NW, ...),
// keep up to four tiles of operands in flight, and the per-wave sums are
// added in wave order through LDS; the epilogue then runs on the reduced
// tile.  Split partial sums (EPI_RAW with S > 1) are added in split order by
// the consumer.
template <int RT, int KT, int NW, int S, int EPI>
__global__ __launch_bounds__(NW * 64) void k_bgemm(const u32x4 *__restrict__ W, const u32x4 *__restrict__ X,
                                                   BEpi ep) {
    constexpr int KTS = KT / S, KTW = KTS / NW, GT = NW * 64;
    static_assert(KT % S == 0 && KTS % NW == 0, "whole k tiles per wave");
    static_assert(S == 1 || EPI == EPI_RAW, "split sums leave the GEMM unrounded");
    constexpr int D = KTW < 4 ? KTW : 4;
    constexpr size_t WSTEP = (size_t)NW * RT * 64, XSTEP = (size_t)NW * 4 * 64;
    __shared__ f32x4 red[NW * RT * 4 * 64];
    __shared__ float lm_v[RT * 4][64];
    __shared__ int lm_i[RT * 4][64];
    __shared__ uint64_t exp2_lds[EPI == EPI_QKVG ? 32 : 1];  // expf's table for the epilogue
    __shared__ f32x4 conv_lds[EPI == EPI_QKVG ? RT * 16 : 1];  // the conv taps of the workgroup's channels
    if constexpr (EPI == EPI_QKVG) fill_exp2_lds_imm(exp2_lds);
    // QKVG: consecutive row blocks on one XCD (workgroups are dealt to the 8
    // XCDs round-robin), so the two 64-byte halves of a conv-tail line are
    // fetched into one XCD's L2 once instead of into two
    const int rb = (EPI == EPI_QKVG && (gridDim.x & 7) == 0)
                       ? (int)((blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3))
                       : (int)blockIdx.x;
    const int t = threadIdx.x, w = t >> 6, l = t & 63, sp = blockIdx.y;
    const int kt0 = sp * KTS + w;
    const u32x4 *wp = W + ((size_t)rb * KT + kt0) * (RT * 64) + l;
    const u32x4 *xp = X + (size_t)kt0 * (4 * 64) + l;

    // QKVG epilogue tasks: four consecutive channels of one stream per
    // thread and pass (4-channel group g of the workgroup's RT * 4, stream
    // q / (RT * 4)), so tails, q/k/v and gate move as 8- and 16-byte
    // accesses.  Each stream's conv tails (three taps of BF16 bits per
    // channel) and the workgroup's taps (into LDS) are read ahead of the
    // weight stream.
    constexpr int CG = RT * 4;
    constexpr int QE = (EPI == EPI_QKVG) ? (64 * CG) / GT : 1;
    static_assert(EPI != EPI_QKVG || (64 * CG) % GT == 0, "whole epilogue tasks per thread");
    const int which = (rb * 16 * RT) / kH, c0 = rb * 16 * RT - which * kH;  // q, k, v, g section
    uint2 qtl[QE][3];
    if constexpr (EPI == EPI_QKVG) {
        if (which < 3 && t < RT * 16)
            conv_lds[t] = *reinterpret_cast<const f32x4 *>(ep.conv_w + ((size_t)which * kH + c0 + t) * 4);
#pragma unroll
        for (int j = 0; j < QE; ++j) {
            const int q = t + GT * j, m = q / CG, c = c0 + 4 * (q % CG);
#pragma unroll
            for (int k = 0; k < 3; ++k) qtl[j][k] = make_uint2(0u, 0u);
            if (which < 3 && m < ep.n_streams) {
                const uint16_t *tl = ep.tails + ((size_t)m * 3 + which) * 3 * kH + c;
#pragma unroll
                for (int k = 0; k < 3; ++k) qtl[j][k] = *reinterpret_cast<const uint2 *>(tl + k * kH);
            }
        }
    }

    f32x4 acc[RT][4];
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int g = 0; g < 4; ++g) acc[r][g] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    u32x4 a[D][RT], b[D][4];
#pragma unroll
    for (int i = 0; i < D; ++i) {
#pragma unroll
        for (int r = 0; r < RT; ++r) a[i][r] = wp[i * WSTEP + r * 64];
#pragma unroll
        for (int g = 0; g < 4; ++g) b[i][g] = xp[i * XSTEP + g * 64];
    }
    // the scheduler keeps every prefetch where it is issued: D k tiles stay
    // in flight instead of one
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < KTW; ++i) {
        const int s = i % D;
#pragma unroll
        for (int r = 0; r < RT; ++r)
#pragma unroll
            for (int g = 0; g < 4; ++g)
                acc[r][g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[s][r]),
                                                                    __builtin_bit_cast(bf16x8, b[s][g]),
                                                                    acc[r][g], 0, 0, 0);
        if (i + D < KTW) {
#pragma unroll
            for (int r = 0; r < RT; ++r) a[s][r] = wp[(i + D) * WSTEP + r * 64];
#pragma unroll
            for (int g = 0; g < 4; ++g) b[s][g] = xp[(i + D) * XSTEP + g * 64];
        }
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int g = 0; g < 4; ++g) red[((w * RT + r) * 4 + g) * 64 + l] = acc[r][g];
    __syncthreads();

    // Task (rt, nq, m): rows rt * 16 + nq * 4 + 0..3 of stream m, held by lane
    // nq * 16 + m % 16 of stream group m / 16 in every wave's D tile.  Every
    // epilogue takes whole tasks (the four rows as one f32x4).
    auto red_index = [&](int rt, int nq, int m) { return (rt * 4 + (m >> 4)) * 64 + nq * 16 + (m & 15); };
    auto reduced = [&](int rt, int nq, int m) {
        const int idx = red_index(rt, nq, m);
        f32x4 v = red[idx];
#pragma unroll
        for (int ww = 1; ww < NW; ++ww) v = v + red[ww * RT * 4 * 64 + idx];
        return v;
    };
    if constexpr (EPI == EPI_RAW || EPI == EPI_STORE || EPI == EPI_LM) {
#pragma unroll
        for (int q = t; q < RT * 4 * 64; q += GT) {
            const int m = q & 63, nq = (q >> 6) & 3, rt = q >> 8;
            const f32x4 v = reduced(rt, nq, m);
            const int row = rb * 16 * RT + rt * 16 + nq * 4;
            if constexpr (EPI == EPI_LM) {
                *reinterpret_cast<f32x4 *>(ep.logits + (size_t)m * ep.n_rows + row) = v;
                float best = -3.402823466e38f;
                int idx = 0;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (v[e] > best) {
                        best = v[e];
                        idx = row + e;
                    }
                lm_v[rt * 4 + nq][m] = best;
                lm_i[rt * 4 + nq][m] = idx;
            } else {
                f32x4 o = v;
                if constexpr (EPI == EPI_STORE) {
                    o.x = rne_bf16(v.x);
                    o.y = rne_bf16(v.y);
                    o.z = rne_bf16(v.z);
                    o.w = rne_bf16(v.w);
                }
                *reinterpret_cast<f32x4 *>(ep.y + ((size_t)sp * 64 + m) * ep.n_rows + row) = o;
            }
        }
    } else if constexpr (EPI == EPI_QKVG) {
#pragma unroll
        for (int j = 0; j < QE; ++j) {
            const int q = t + GT * j, g = q % CG, m = q / CG, c = c0 + 4 * g;
            if (m >= ep.n_streams) continue;
            // channels c..c+3 are rows 4 (g % 4) .. of row tile g / 4
            const f32x4 v = reduced(g >> 2, g & 3, m);
            const float raw[4] = {rne_bf16(v.x), rne_bf16(v.y), rne_bf16(v.z), rne_bf16(v.w)};
            if (which < 3) {
                // gdn_depthwise_conv_silu_head_kind, gdn_model.cpp:1543-1667
                uint16_t *tl = ep.tails + ((size_t)m * 3 + which) * 3 * kH + c;
                const uint32_t tw[3][2] = {{qtl[j][0].x, qtl[j][0].y}, {qtl[j][1].x, qtl[j][1].y},
                                           {qtl[j][2].x, qtl[j][2].y}};
                float o[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int sh = 16 * (e & 1);
                    const f32x4 cw = conv_lds[4 * g + e];
                    const float t0 = bf16_bits_to_f32((uint16_t)(tw[0][e >> 1] >> sh));
                    const float t1 = bf16_bits_to_f32((uint16_t)(tw[1][e >> 1] >> sh));
                    const float t2 = bf16_bits_to_f32((uint16_t)(tw[2][e >> 1] >> sh));
                    const float sum = t0 * cw.x + t1 * cw.y + t2 * cw.z + raw[e] * cw.w;
                    o[e] = rne_bf16(silu_ref(sum, Exp2Lds{exp2_lds}));
                }
                // the tails shift by one tap: (t1, t2, raw)
                *reinterpret_cast<uint2 *>(tl) = qtl[j][1];
                *reinterpret_cast<uint2 *>(tl + kH) = qtl[j][2];
                *reinterpret_cast<uint2 *>(tl + 2 * kH) =
                    make_uint2((uint32_t)bf16_hi(raw[0]) | ((uint32_t)bf16_hi(raw[1]) << 16),
                               (uint32_t)bf16_hi(raw[2]) | ((uint32_t)bf16_hi(raw[3]) << 16));
                *reinterpret_cast<f32x4 *>(ep.qkv + ((size_t)m * 3 + which) * kH + c) =
                    (f32x4){o[0], o[1], o[2], o[3]};
            } else {
                *reinterpret_cast<f32x4 *>(ep.gate + (size_t)m * kH + c) = (f32x4){raw[0], raw[1], raw[2], raw[3]};
                *reinterpret_cast<f32x4 *>(ep.sgate + (size_t)m * kH + c) =
                    (f32x4){sigmoid_ref(raw[0], Exp2Lds{exp2_lds}), sigmoid_ref(raw[1], Exp2Lds{exp2_lds}),
                            sigmoid_ref(raw[2], Exp2Lds{exp2_lds}), sigmoid_ref(raw[3], Exp2Lds{exp2_lds})};
            }
        }
    }
    if constexpr (EPI == EPI_LM) {
        __syncthreads();
        if (t < 64) {
            // row quads in index order: strict '>' keeps the lowest index of
            // equal maxima (NaN never wins)
            float best = lm_v[0][t];
            int idx = lm_i[0][t];
#pragma unroll
            for (int q = 1; q < RT * 4; ++q)
                if (lm_v[q][t] > best) {
                    best = lm_v[q][t];
                    idx = lm_i[q][t];
                }
            ep.part_val[(size_t)rb * 64 + t] = best;
            ep.part_idx[(size_t)rb * 64 + t] = idx;
        }
    }
}

// ------------------------------------------------------------ gate/up
//
// 5632 channels over 256 workgroups, one per CU: workgroup b owns channels
// 22 b .. 22 b + 21, i.e. 44 rows in three row tiles: the gate rows of its
// first 16 channels, their up rows, and a 12-row tile with the gate then the
// up rows of the last 6 (rows 12..15 of that tile stay zero).  Whole 16-row
// pairs (32 rows per workgroup) give 352 workgroups, i.e. two on some CUs,
// and every workgroup reads all 64 streams' activations beside its rows.
constexpr int kGuCh = 22;                // channels per gate/up workgroup
constexpr int kGuWgs = kI / kGuCh;       // 256
constexpr int kGuTail2 = 2 * (kGuCh - 16);     // rows of the third tile (12)
constexpr int kGuTileU4 = 128 + 4 * kGuTail2;  // 16-byte entries per k tile
constexpr int kGuWaves = 4;                    // waves per gate/up workgroup
static_assert(kGuWgs * kGuCh == kI && kGuCh > 16 && kGuCh <= 24 && (kGuCh % 2) == 0, "gate/up split");

// One k tile of the layout: tile 0 lane l = (row l % 16, columns 8 (l / 16)..),
// tile 1 likewise, the 12-row tile's entry (quarter kq, row r) at 128 + kq * 12 + r.
// The NW waves split the 64 k tiles as k_bgemm's do (wave w: w, w + NW, ...)
// and the per-wave sums are added in wave order, so each channel's sums are
// those of k_bgemm's 16-channel pairing with the same NW.
template <int NW>
__global__ __launch_bounds__(NW * 64) void k_bgu(const u32x4 *__restrict__ W, const u32x4 *__restrict__ X,
                                                 uint16_t *__restrict__ x_next, int n_streams) {
    constexpr int RT = 3, KT = kKtH, KTW = KT / NW, GT = NW * 64;
    static_assert(KT % NW == 0, "whole k tiles per wave");
    constexpr int D = KTW < 4 ? KTW : 4;
    constexpr size_t WSTEP = (size_t)NW * kGuTileU4, XSTEP = (size_t)NW * 4 * 64;
    __shared__ f32x4 red[NW * RT * 4 * 64];
    __shared__ uint64_t exp2_lds[32];  // expf's table for the SwiGLU epilogue
    const int t = threadIdx.x, w = t >> 6, l = t & 63, rb = blockIdx.x;
    fill_exp2_lds_imm(exp2_lds);
    // the 12-row tile: lanes of rows 12..15 read entry 0 (in bounds) and
    // zero it
    const bool p2 = (l & 15) < kGuTail2;
    const int o2 = 128 + (p2 ? (l >> 4) * kGuTail2 + (l & 15) : 0);
    const u32x4 *wp = W + ((size_t)rb * KT + w) * kGuTileU4;
    const u32x4 *xp = X + (size_t)w * (4 * 64) + l;
    const u32x4 zero = {0u, 0u, 0u, 0u};

    f32x4 acc[RT][4];
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int g = 0; g < 4; ++g) acc[r][g] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    u32x4 a[D][RT], b[D][4];
#pragma unroll
    for (int i = 0; i < D; ++i) {
        a[i][0] = wp[i * WSTEP + l];
        a[i][1] = wp[i * WSTEP + 64 + l];
        a[i][2] = wp[i * WSTEP + o2];
#pragma unroll
        for (int g = 0; g < 4; ++g) b[i][g] = xp[i * XSTEP + g * 64];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < KTW; ++i) {
        const int s = i % D;
        if (!p2) a[s][2] = zero;
#pragma unroll
        for (int r = 0; r < RT; ++r)
#pragma unroll
            for (int g = 0; g < 4; ++g)
                acc[r][g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[s][r]),
                                                                    __builtin_bit_cast(bf16x8, b[s][g]),
                                                                    acc[r][g], 0, 0, 0);
        if (i + D < KTW) {
            a[s][0] = wp[(i + D) * WSTEP + l];
            a[s][1] = wp[(i + D) * WSTEP + 64 + l];
            a[s][2] = wp[(i + D) * WSTEP + o2];
#pragma unroll
            for (int g = 0; g < 4; ++g) b[s][g] = xp[(i + D) * XSTEP + g * 64];
        }
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int g = 0; g < 4; ++g) red[((w * RT + r) * 4 + g) * 64 + l] = acc[r][g];
    __syncthreads();

    // rows 4 nq .. 4 nq + 3 of tile r for stream m: lane nq * 16 + m % 16 of
    // stream group m / 16 in every wave's tile, the waves added in order
    auto val4 = [&](int r, int nq, int m) {
        const int idx = (r * 4 + (m >> 4)) * 64 + nq * 16 + (m & 15);
        f32x4 v = red[idx];
#pragma unroll
        for (int ww = 1; ww < NW; ++ww) v = v + red[ww * RT * 4 * 64 + idx];
        return v;
    };
    // gemv32_store SwiGLU branch, gdn_model.cpp:4751-4767, for one channel
    // (its gate g and up u as the GEMM left them)
    auto swiglu = [&](float g, float u) {
        return bf16_daz_bits(rne_bf16(silu_ref(rne_bf16(g), Exp2Lds{exp2_lds}) * rne_bf16(u)));
    };
    static_assert(kGuCh == 22 && GT == 256, "16 + 6 channels; 256 + 192 tasks over four waves");
    // channels 4 nq .. 4 nq + 3 (gate rows of tile 0, up rows of tile 1):
    // task (stream m, nq), thread 4 m + nq
    {
        const int m = t >> 2, nq = t & 3;
        if (m < n_streams) {
            const f32x4 g = val4(0, nq, m), u = val4(1, nq, m);
            const uint32_t lo = swiglu(g.x, u.x) | (swiglu(g.y, u.y) << 16);
            const uint32_t hi = swiglu(g.z, u.z) | (swiglu(g.w, u.w) << 16);
            const int k0 = rb * kGuCh + 4 * nq;  // even: pairs never straddle an 8-column group
            if ((k0 & 3) == 0) {
                *reinterpret_cast<uint2 *>(x_next + xt_index(m, k0, kI)) = make_uint2(lo, hi);
            } else {
                *reinterpret_cast<uint32_t *>(x_next + xt_index(m, k0, kI)) = lo;
                *reinterpret_cast<uint32_t *>(x_next + xt_index(m, k0 + 2, kI)) = hi;
            }
        }
    }
    // channels 16 + 2 p, 17 + 2 p (gate rows 2 p, 2 p + 1 and up rows
    // 2 p + 6, 2 p + 7 of tile 2): task (stream m, p), thread 64 + 3 m + p
    if (t >= 64) {
        const int q = t - 64, m = q / 3, p = q - 3 * m;
        if (m < n_streams) {
            const int rg = 2 * p, ru = 2 * p + 6;
            const f32x4 gv = val4(2, rg >> 2, m), uv = val4(2, ru >> 2, m);
            const float g0 = (rg & 3) ? gv.z : gv.x, g1 = (rg & 3) ? gv.w : gv.y;
            const float u0 = (ru & 3) ? uv.z : uv.x, u1 = (ru & 3) ? uv.w : uv.y;
            *reinterpret_cast<uint32_t *>(x_next + xt_index(m, rb * kGuCh + 16 + 2 * p, kI)) =
                swiglu(g0, u0) | (swiglu(g1, u1) << 16);
        }
    }
}

// Per-stream merge of the LM head's per-workgroup results (in index order):
// strict '>' within a thread's increasing blocks, then larger value / lower
// index across threads -- the reference's first-maximum scan.
__global__ __launch_bounds__(kT) void k_bargmax(const float *__restrict__ part_val,
                                                const int *__restrict__ part_idx, int n_blocks,
                                                int *__restrict__ tok_out) {
    __shared__ float bv[4];
    __shared__ int bi[4];
    const int m = blockIdx.x, t = threadIdx.x;
    float best = -3.402823466e38f;
    int idx = 0;
    for (int i = t; i < n_blocks; i += kT) {
        const float v = part_val[(size_t)i * 64 + m];
        if (v > best) {
            best = v;
            idx = part_idx[(size_t)i * 64 + m];
        }
    }
#pragma unroll
    for (int s = 1; s < 64; s <<= 1) {
        const float ov = __shfl_xor(best, s);
        const int oi = __shfl_xor(idx, s);
        if (ov > best || (ov == best && oi < idx)) {
            best = ov;
            idx = oi;
        }
    }
    if ((t & 63) == 0) {
        bv[t >> 6] = best;
        bi[t >> 6] = idx;
    }
    __syncthreads();
    if (t == 0) {
        for (int i = 1; i < 4; ++i)
            if (bv[i] > best || (bv[i] == best && bi[i] < idx)) {
                best = bv[i];
                idx = bi[i];
            }
        tok_out[m] = idx;
    }
}

// ------------------------------------------------------ per-stream kernels

struct BNorm {
    const float *h_in;     // [64][kH] residual stream
    float *h_out;          // h_in, or (AB, several workgroups per stream) the other residual buffer
    const float *y;        // [splits][64][kH] partial sums: h = R(h + R(sum)) first
    const uint16_t *emb;   // embedding rows (BF16): h = R(emb[tok[m]]) (EMBED)
    const int *tok;
    const float *w;        // norm weight [kH]
    uint16_t *x_out;       // X tiles of the next projection
    float *xn_out;         // optional [64][kH] copy of the normalized vector
    const float *ab_w;     // a_proj (8 x kH) then b_proj (8 x kH) (AB)
    const float *a_log;
    const float *dt_bias;
    float *bd;             // [64][16]: beta, decay per head
    float eps;
};

// Per stream: the residual add (or embedding import), the RMSNorm in chunk
// order (gdn_rmsnorm_rows_bf16 / gdn_residual_rmsnorm_bf16,
// gdn_model.cpp:1394-1474, :3351-3450) and, before an attention block, the
// tiny a/b rows and beta/decay (gdn_gemv_tiny_ab :1501-1536, :2461-2465).
// Thread t holds elements 8t..8t+7; a 16-element chunk is the sequential sum
// of thread 2c's eight squares continued by thread 2c + 1.  SPLITS partial
// sums of the preceding projection are added in split order (0: no residual
// add; EMBED: the embedding row instead).  Without AB one workgroup per
// stream updates the residual in place.  With AB, grid (streams, kAbSplit):
// workgroup j repeats the norm and runs the a/b rows of heads
// kNH / kAbSplit * j .. (a 32 KB slice of the 128 KB of rows, requested
// before the norm's first wait on memory); workgroup 0 alone writes the
// residual, to h_out != h_in, and the X tiles.
constexpr int kAbSplit = 4;
constexpr int kAbHeads = kNH / kAbSplit;  // heads per a/b workgroup
static_assert(kNH % kAbSplit == 0 && (2 * kAbHeads * kH) % (4 * kT) == 0 && 2 * kAbHeads <= kT,
              "whole heads per a/b workgroup, whole 16-byte row pieces per thread");
template <int SPLITS, bool EMBED, bool AB>
__global__ __launch_bounds__(kT) void k_bnorm(BNorm p) {
    constexpr int ABR = 2 * kAbHeads;  // a/b rows per workgroup: a rows, then b rows
    __shared__ __attribute__((aligned(16))) float xs[kH];
    __shared__ __attribute__((aligned(16))) float cs[kH / 16];
    __shared__ __attribute__((aligned(16))) float tab[ABR][64][2];
    __shared__ float abv[ABR];
    __shared__ float scale_s;
    const int m = blockIdx.x, t = threadIdx.x, e0 = 8 * t;
    const int j = AB ? (int)blockIdx.y : 0;
    const bool writer = j == 0;
    const f32x4 *w4 = reinterpret_cast<const f32x4 *>(p.w + e0);
    const f32x4 wa = w4[0], wb = w4[1];
    float hv[8];
    if constexpr (EMBED) {
        const u32x4 raw = *reinterpret_cast<const u32x4 *>(p.emb + (size_t)p.tok[m] * kH + e0);
        const uint32_t wv[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            hv[2 * j] = rne_bf16(u2f(wv[j] << 16));
            hv[2 * j + 1] = rne_bf16(u2f(wv[j] & 0xffff0000u));
        }
    } else {
        const f32x4 *h4 = reinterpret_cast<const f32x4 *>(p.h_in + (size_t)m * kH + e0);
        const f32x4 a0 = h4[0], a1 = h4[1];
        hv[0] = a0.x; hv[1] = a0.y; hv[2] = a0.z; hv[3] = a0.w;
        hv[4] = a1.x; hv[5] = a1.y; hv[6] = a1.z; hv[7] = a1.w;
        if constexpr (SPLITS > 0) {
            // the projection's split sums in split order, then its rounding
            f32x4 yp[SPLITS][2];
#pragma unroll
            for (int sp = 0; sp < SPLITS; ++sp) {
                const f32x4 *y4 = reinterpret_cast<const f32x4 *>(p.y + ((size_t)sp * kMaxB + m) * kH + e0);
                yp[sp][0] = y4[0];
                yp[sp][1] = y4[1];
            }
            f32x4 y0 = yp[0][0], y1 = yp[0][1];
#pragma unroll
            for (int sp = 1; sp < SPLITS; ++sp) {
                y0 = y0 + yp[sp][0];
                y1 = y1 + yp[sp][1];
            }
            const float yv[8] = {y0.x, y0.y, y0.z, y0.w, y1.x, y1.y, y1.z, y1.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) hv[e] = rne_bf16(hv[e] + rne_bf16(yv[e]));
        }
    }
    // the a/b rows are requested behind the operands of the norm (loads
    // return in order)
    // local row r: a row of head kAbHeads j + r (r < kAbHeads), else the b
    // row of head kAbHeads j + r - kAbHeads
    auto ab_row = [&](int r) { return r < kAbHeads ? kAbHeads * j + r : kNH + kAbHeads * j + r - kAbHeads; };
    constexpr int ABN = AB ? ABR * kH / (4 * kT) : 1;
    f32x4 wq[ABN];
    if constexpr (AB) {
#pragma unroll
        for (int i = 0; i < ABN; ++i) {
            const int q = t + kT * i, grp = q >> 3, sub = q & 7;
            wq[i] = *reinterpret_cast<const f32x4 *>(p.ab_w + (size_t)ab_row(grp >> 6) * kH + 32 * (grp & 63) +
                                                     4 * sub);
        }
    }
    if ((EMBED || SPLITS > 0) && writer) {
        f32x4 *d = reinterpret_cast<f32x4 *>(p.h_out + (size_t)m * kH + e0);
        d[0] = (f32x4){hv[0], hv[1], hv[2], hv[3]};
        d[1] = (f32x4){hv[4], hv[5], hv[6], hv[7]};
    }
    // chunk sums: the even thread's partial continues in the odd thread
    float part = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) part += hv[e] * hv[e];
    const float lead = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(part), 0xB1, 0xf, 0xf, false));
    if (t & 1) {
        float s = lead;
#pragma unroll
        for (int e = 0; e < 8; ++e) s += hv[e] * hv[e];
        cs[t >> 1] = s;
    }
    __syncthreads();
    if (t == 0) {
        // every chunk sum read ahead of the sequential adds
        float v[kH / 16];
#pragma unroll
        for (int c = 0; c < kH / 64; ++c) {
            const f32x4 q = reinterpret_cast<const f32x4 *>(cs)[c];
            v[4 * c] = q.x;
            v[4 * c + 1] = q.y;
            v[4 * c + 2] = q.z;
            v[4 * c + 3] = q.w;
        }
        float sum = 0.0f;
#pragma unroll
        for (int c = 0; c < kH / 16; ++c) sum += v[c];
        scale_s = 1.0f / __builtin_sqrtf(sum / (float)kH + p.eps);
    }
    __syncthreads();
    const float sc = scale_s;
    const float wv[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
    float xv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) xv[e] = rne_bf16(hv[e] * sc * wv[e]);
    if (writer) store_x8(p.x_out, m, e0, xv);
    if (p.xn_out && writer) {
        f32x4 *d = reinterpret_cast<f32x4 *>(p.xn_out + (size_t)m * kH + e0);
        d[0] = (f32x4){xv[0], xv[1], xv[2], xv[3]};
        d[1] = (f32x4){xv[4], xv[5], xv[6], xv[7]};
    }
    if constexpr (AB) {
        {
            f32x4 *d = reinterpret_cast<f32x4 *>(xs + e0);
            d[0] = (f32x4){xv[0], xv[1], xv[2], xv[3]};
            d[1] = (f32x4){xv[4], xv[5], xv[6], xv[7]};
        }
        __syncthreads();
        // Eight lanes per (local row, 32-column beat), four products each:
        // lanes 0-3 form tree16 of the lower half, lanes 4-7 of the upper
        // (pairs, then lane pairs, then lane quads), so a wave's loads cover
        // eight consecutive beats of one row.
#pragma unroll
        for (int i = 0; i < ABN; ++i) {
            const int q = t + kT * i, grp = q >> 3, sub = q & 7;
            const f32x4 xq = *reinterpret_cast<const f32x4 *>(xs + 32 * (grp & 63) + 4 * sub);
            const f32x4 w = wq[i];
            float s = (xq.x * w.x + xq.y * w.y) + (xq.z * w.z + xq.w * w.w);
            s = quad_sum(s);
            if ((sub & 3) == 0) tab[grp >> 6][grp & 63][sub >> 2] = s;
        }
        __syncthreads();
        if (t < ABR) {
            float v[128];
#pragma unroll
            for (int i = 0; i < 32; ++i) {
                const f32x4 q = reinterpret_cast<const f32x4 *>(&tab[t][0][0])[i];
                v[4 * i] = q.x;
                v[4 * i + 1] = q.y;
                v[4 * i + 2] = q.z;
                v[4 * i + 3] = q.w;
            }
            float acc = 0.0f;
#pragma unroll
            for (int bt = 0; bt < 64; ++bt) acc = (acc + v[2 * bt]) + v[2 * bt + 1];
            abv[t] = rne_bf16(acc);
        }
        __syncthreads();
        if (t < kAbHeads) {
            const int hd = kAbHeads * j + t;
            float beta, decay;
            head_scalars(abv[t], abv[kAbHeads + t], p.a_log[hd], p.dt_bias[hd], beta, decay);
            p.bd[m * 16 + 2 * hd] = beta;
            p.bd[m * 16 + 2 * hd + 1] = decay;
        }
    }
}

// The a/b rows and beta/decay of kPabTok tokens per workgroup, from their
// normalised inputs (the prefill's split of k_bnorm's AB part, whose
// workgroups each re-read their 32 KB of rows): grid (kAbSplit, ceil(n /
// kPabTok)).  Workgroup j loads its four rows once.  Per token the thread
// tasks, products, quad sums, the 64-beat chains and the head scalars are
// k_bnorm's, so every value is the step's.
constexpr int kPabTok = 16;
__global__ __launch_bounds__(kT) void k_pab(const float *__restrict__ xn, int n, const float *__restrict__ ab_w,
                                            const float *__restrict__ a_log, const float *__restrict__ dt_bias,
                                            float *__restrict__ bd) {
    constexpr int ABR = 2 * kAbHeads, ABN = ABR * kH / (4 * kT);
    static_assert(kPabTok * ABR <= kT, "one chain thread per (token, row)");
    __shared__ __attribute__((aligned(16))) float tab[kPabTok][ABR][64][2];
    __shared__ float abv[kPabTok][ABR];
    __shared__ uint64_t exp2_lds[32];
    const int j = blockIdx.x, m0 = (int)blockIdx.y * kPabTok, t = threadIdx.x;
    fill_exp2_lds_imm(exp2_lds);
    // local row r: the a row of head kAbHeads j + r (r < kAbHeads), else the
    // b row of head kAbHeads j + r - kAbHeads
    auto ab_row = [&](int r) { return r < kAbHeads ? kAbHeads * j + r : kNH + kAbHeads * j + r - kAbHeads; };
    f32x4 wq[ABN];
#pragma unroll
    for (int i = 0; i < ABN; ++i) {
        const int q = t + kT * i, grp = q >> 3, sub = q & 7;
        wq[i] = *reinterpret_cast<const f32x4 *>(ab_w + (size_t)ab_row(grp >> 6) * kH + 32 * (grp & 63) + 4 * sub);
    }
    // PG tokens' inputs requested together (a token past the segment's end
    // re-reads its last one, unused), then their products
    constexpr int PG = 4;
    static_assert(kPabTok % PG == 0, "whole token groups");
    for (int mg = 0; mg < kPabTok && m0 + mg < n; mg += PG) {
        f32x4 xq[PG][ABN];
#pragma unroll
        for (int g = 0; g < PG; ++g) {
            const int m = m0 + mg + g < n ? m0 + mg + g : n - 1;
            const float *x = xn + (size_t)m * kH;
#pragma unroll
            for (int i = 0; i < ABN; ++i) {
                const int q = t + kT * i, grp = q >> 3, sub = q & 7;
                xq[g][i] = *reinterpret_cast<const f32x4 *>(x + 32 * (grp & 63) + 4 * sub);
            }
        }
#pragma unroll
        for (int g = 0; g < PG; ++g) {
#pragma unroll
            for (int i = 0; i < ABN; ++i) {
                const int q = t + kT * i, grp = q >> 3, sub = q & 7;
                const f32x4 w = wq[i], x = xq[g][i];
                float s = (x.x * w.x + x.y * w.y) + (x.z * w.z + x.w * w.w);
                s = quad_sum(s);
                if ((sub & 3) == 0) tab[mg + g][grp >> 6][grp & 63][sub >> 2] = s;
            }
        }
    }
    __syncthreads();
    if (t < kPabTok * ABR) {
        const int mt = t / ABR, r = t % ABR;
        if (m0 + mt < n) {
            float v[128];
#pragma unroll
            for (int i = 0; i < 32; ++i) {
                const f32x4 q = reinterpret_cast<const f32x4 *>(&tab[mt][r][0][0])[i];
                v[4 * i] = q.x;
                v[4 * i + 1] = q.y;
                v[4 * i + 2] = q.z;
                v[4 * i + 3] = q.w;
            }
            float acc = 0.0f;
#pragma unroll
            for (int bt = 0; bt < 64; ++bt) acc = (acc + v[2 * bt]) + v[2 * bt + 1];
            abv[mt][r] = rne_bf16(acc);
        }
    }
    __syncthreads();
    if (t < kPabTok * kAbHeads) {
        const int mt = t / kAbHeads, hh = t % kAbHeads, m = m0 + mt;
        if (m < n) {
            const int hd = kAbHeads * j + hh;
            float beta, decay;
            head_scalars(abv[mt][hh], abv[mt][kAbHeads + hh], a_log[hd], dt_bias[hd], beta, decay,
                         Exp2Lds{exp2_lds});
            bd[m * 16 + 2 * hd] = beta;
            bd[m * 16 + 2 * hd + 1] = decay;
        }
    }
}

// Per (head, stream): the output RMSNorm times the gate and sigmoid(gate)
// (gdn_output_norm_and_gate, gdn_model.cpp:3226-3349) into X tiles, for
// streams (or prefill tokens) PT y .. PT y + PT - 1 of n: every input of
// the workgroup's PT streams is requested at its start (a stream past n
// re-reads stream n - 1, unused), so they share one memory latency.
template <int PT>
__global__ __launch_bounds__(kT) void k_bonorm(const float *__restrict__ attn, const float *__restrict__ gate,
                                               const float *__restrict__ sgate, const float *__restrict__ w,
                                               float eps, uint16_t *__restrict__ x_out, int n) {
    static_assert(PT * (kHD / 8) <= kT && kT == kHD, "a thread per channel; one X store task per thread");
    __shared__ float as[PT][kHD];
    __shared__ float cs[PT][kHD / 16];
    __shared__ float xs[PT][kHD];
    __shared__ float scale_s[PT];
    const int h = blockIdx.x, m0 = (int)blockIdx.y * PT, t = threadIdx.x, c = h * kHD + t;
    float a[PT], gt[PT], sg[PT];
#pragma unroll
    for (int i = 0; i < PT; ++i) {
        const size_t o = (size_t)(m0 + i < n ? m0 + i : n - 1) * kH + c;
        a[i] = attn[o];
        gt[i] = gate[o];
        sg[i] = sgate[o];
    }
    const float wt = w[t];
#pragma unroll
    for (int i = 0; i < PT; ++i) as[i][t] = a[i];
    __syncthreads();
    if (t < PT * (kHD / 16)) {
        const int i = t / (kHD / 16), r = t % (kHD / 16);
        float s = 0.0f;
#pragma unroll
        for (int kk = 0; kk < 16; ++kk) {
            const float v = as[i][16 * r + kk];
            s += v * v;
        }
        cs[i][r] = s;
    }
    __syncthreads();
    if (t < PT) {
        float v[kHD / 16];
#pragma unroll
        for (int i = 0; i < kHD / 16; ++i) v[i] = cs[t][i];
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < kHD / 16; ++i) sum += v[i];
        scale_s[t] = 1.0f / __builtin_sqrtf(sum / (float)kHD + eps);
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < PT; ++i) xs[i][t] = rne_bf16(a[i] * scale_s[i] * wt * gt[i] * sg[i]);
    __syncthreads();
    if (t < PT * (kHD / 8)) {
        const int i = t / (kHD / 8), j = t % (kHD / 8);
        if (m0 + i < n) store_x8(x_out, m0 + i, h * kHD + 8 * j, xs[i] + 8 * j);
    }
}
constexpr int kOnTok = 4;  // prefill tokens per output-norm workgroup

// The recurrence of one (head, stream, CW-column group) per workgroup of
// 2 CW threads, with the batch-1 arithmetic (gdn_island_prep / read /
// update, gdn_model.cpp:2376-2933).  Wave w owns state column
// c0 + 64 (w % (CW / 64)) + lane and rows 128 (w / (CW / 64)) .. + 127,
// held in registers from load to store: the first half of the waves run
// the r and p chains over rows 0..127, hand the partial sums to the second
// half through LDS, which continue over rows 128..255 (the chain order is
// j = 0..255 as in the reference) and form delta and o; every wave then
// writes its rows of S' = decay * S + kn (x) delta.  The q/k norms and alpha
// use the batch-1 tree order; every column group of a head computes them.
// 128-column groups (256 threads) leave room for three workgroups per CU,
// so one group's stores overlap another's loads.
template <int CW>
__global__ __launch_bounds__(2 * CW) void k_brecur(const float *__restrict__ qkv, const float *__restrict__ bd,
                                                   float *__restrict__ state, float *__restrict__ attn) {
    static_assert(CW == 128 || CW == 256, "column groups of 128 or 256");
    constexpr int RH = kHD / 2;   // rows per wave
    constexpr int WPR = CW / 64;  // waves per 128-row half
    __shared__ float qn[kHD], kn[kHD], rpart[CW], ppart[CW], dl[CW];
    __shared__ float red[8], red2[4];
    const int cg = blockIdx.x % (kHD / CW), h = blockIdx.x / (kHD / CW), m = blockIdx.y;
    const int t = threadIdx.x, w = t >> 6, lane = t & 63;
    const int lc = (w % WPR) * 64 + lane, col = cg * CW + lc, r0 = (w / WPR) * RH;
    const float *qp = qkv + (size_t)m * 3 * kH + h * kHD;
    float *S = state + (size_t)m * kLayerState + (size_t)h * kHD * kHD + col;
    float sv[RH];
#pragma unroll
    for (int j = 0; j < RH; ++j) sv[j] = S[(size_t)(r0 + j) * kHD];
    const float beta = bd[m * 16 + 2 * h], decay = bd[m * 16 + 2 * h + 1];
    float q = 0.0f, k = 0.0f;
    if (t < kHD) {
        q = qp[t];
        k = qp[kH + t];
        const float qs = wave_tree64(q * q), ks = wave_tree64(k * k);
        if (lane == 0) {
            red[w] = qs;
            red[4 + w] = ks;
        }
    }
    __syncthreads();
    if (t < kHD) {
        const float q_sq = (red[0] + red[1]) + (red[2] + red[3]);
        const float k_sq = (red[4] + red[5]) + (red[6] + red[7]);
        const float qv = q * (1.0f / __builtin_sqrtf(q_sq + 1e-6f));
        const float kv = k * (1.0f / __builtin_sqrtf(k_sq + 1e-6f));
        qn[t] = qv;
        kn[t] = kv;
        const float qk = wave_tree64(qv * kv);
        if (lane == 0) red2[w] = qk;
    }
    __syncthreads();
    if (w < WPR) {
        float r = 0.0f, p = 0.0f;
#pragma unroll
        for (int j = 0; j < RH; ++j) {
            r = r + sv[j] * kn[j];
            p = p + sv[j] * qn[j];
        }
        rpart[lc] = r;
        ppart[lc] = p;
    }
    __syncthreads();
    if (w >= WPR) {
        float r = rpart[lc], p = ppart[lc];
#pragma unroll
        for (int j = 0; j < RH; ++j) {
            r = r + sv[j] * kn[RH + j];
            p = p + sv[j] * qn[RH + j];
        }
        const float alpha = (red2[0] + red2[1]) + (red2[2] + red2[3]);
        const float delta = beta * (qp[2 * kH + col] - decay * r);
        const float o = 0.0625f * (decay * p + alpha * delta);
        dl[lc] = delta;
        attn[(size_t)m * kH + h * kHD + col] = rne_bf16(o);
    }
    __syncthreads();
    const float d = dl[lc];
#pragma unroll
    for (int j = 0; j < RH; ++j) S[(size_t)(r0 + j) * kHD] = decay * sv[j] + kn[r0 + j] * d;
}

// ---------------------------------------------------------------- prefill
//
// A prompt runs through one stream's state in chunks of up to 64 tokens, the
// tokens taking the place of the streams: each layer's projections take the
// whole chunk (the same GEMMs and reduction order as the step), the causal
// conv reads its taps from the neighbouring tokens of the chunk, and one
// workgroup per head runs the recurrence over the chunk's tokens in order
// with the state held in registers.  Every token sees the arithmetic of a
// multi-stream step, so a prefill of n tokens equals n steps bit for bit.

// The causal conv of one 64-channel block over 64 tokens of a segment of n:
// grid (4 kH / 64, ceil(n / 64)), thread 16 r + j on channels 4 j .. 4 j + 3
// of the block and tokens r, r + 16, r + 32, r + 48 (16-byte loads and
// stores; the four loads in flight together).  raw is [n][4 kH] (the
// unrounded q, k, v, g sums); the tails are the prefilled stream's for this
// layer, [q,k,v][3 oldest..newest][kH].  Token m's window is (s[m], s[m+1],
// s[m+2]) and its input s[m+3] in the sequence s = tails ++ R(raw[0..n));
// the new tails are s[n], s[n+1], s[n+2].  Only the first token block reads
// the old tails, and it writes the new ones after that read.
constexpr int kConvT = 256;                  // threads per conv workgroup
constexpr int kConvR = 16 * kMaxB / kConvT;  // tokens per thread
__global__ __launch_bounds__(kConvT) void k_pconv(const float *__restrict__ raw, int n, uint16_t *__restrict__ tails,
                                                  const float *__restrict__ conv_w, float *__restrict__ qkv,
                                                  float *__restrict__ gate, float *__restrict__ sgate) {
    static_assert(kConvR * kConvT == 16 * kMaxB && kConvT >= 64, "16 lanes of 4 channels x kMaxB tokens");
    constexpr int MS = kConvT / 16;  // token stride between a thread's tokens
    __shared__ __attribute__((aligned(16))) float xs[kMaxB + 3][64];
    __shared__ uint64_t exp2_lds[32];  // expf's table, read per SiLU / sigmoid
    const int row0 = blockIdx.x * 64, t = threadIdx.x, mr = t >> 4, c4 = 4 * (t & 15);
    const int m0 = (int)blockIdx.y * kMaxB, nb = n - m0 < kMaxB ? n - m0 : kMaxB;
    fill_exp2_lds_imm(exp2_lds);
    const Exp2Lds tab{exp2_lds};
    const int which = row0 / kH, cb = row0 - which * kH;  // section and its first channel
    // tokens m0 + mr + MS i: raw sums of channels cb + c4 .. + 3.  Tokens
    // past the segment load its last token (in bounds, unused), so every
    // load is unconditional and all are in flight at once.
    f32x4 rr[kConvR];
#pragma unroll
    for (int i = 0; i < kConvR; ++i) {
        const int m = mr + MS * i < nb ? mr + MS * i : nb - 1;
        const f32x4 r = *reinterpret_cast<const f32x4 *>(raw + (size_t)(m0 + m) * 4 * kH + row0 + c4);
        rr[i] = (f32x4){rne_bf16(r.x), rne_bf16(r.y), rne_bf16(r.z), rne_bf16(r.w)};
    }
    if (which < 3) {
        uint16_t *tl = tails + (size_t)which * 3 * kH + cb;
        const f32x4 *cw4 = reinterpret_cast<const f32x4 *>(conv_w + ((size_t)which * kH + cb + c4) * 4);
        const f32x4 cw[4] = {cw4[0], cw4[1], cw4[2], cw4[3]};
        if (t < 64) {
            if (m0 == 0) {
                xs[0][t] = bf16_bits_to_f32(tl[t]);
                xs[1][t] = bf16_bits_to_f32(tl[kH + t]);
                xs[2][t] = bf16_bits_to_f32(tl[2 * kH + t]);
            } else {
#pragma unroll
                for (int i = 0; i < 3; ++i) xs[i][t] = rne_bf16(raw[(size_t)(m0 - 3 + i) * 4 * kH + row0 + t]);
            }
        }
#pragma unroll
        for (int i = 0; i < kConvR; ++i)
            if (mr + MS * i < nb) *reinterpret_cast<f32x4 *>(&xs[3 + mr + MS * i][c4]) = rr[i];
        __syncthreads();
#pragma unroll
        for (int i = 0; i < kConvR; ++i) {
            const int m = mr + MS * i;
            if (m >= nb) break;
            // gdn_depthwise_conv_silu_head_kind, gdn_model.cpp:1543-1667
            const f32x4 x0 = *reinterpret_cast<const f32x4 *>(&xs[m][c4]);
            const f32x4 x1 = *reinterpret_cast<const f32x4 *>(&xs[m + 1][c4]);
            const f32x4 x2 = *reinterpret_cast<const f32x4 *>(&xs[m + 2][c4]);
            const f32x4 x3 = *reinterpret_cast<const f32x4 *>(&xs[m + 3][c4]);
            f32x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float sum = x0[e] * cw[e].x + x1[e] * cw[e].y + x2[e] * cw[e].z + x3[e] * cw[e].w;
                o[e] = rne_bf16(silu_ref(sum, tab));
            }
            *reinterpret_cast<f32x4 *>(qkv + ((size_t)(m0 + m) * 3 + which) * kH + cb + c4) = o;
        }
        if (t < 64 && m0 == 0) {
            if (n <= kMaxB) {
                tl[t] = bf16_hi(xs[n][t]);
                tl[kH + t] = bf16_hi(xs[n + 1][t]);
                tl[2 * kH + t] = bf16_hi(xs[n + 2][t]);
            } else {
#pragma unroll
                for (int i = 0; i < 3; ++i)
                    tl[i * kH + t] = bf16_hi(rne_bf16(raw[(size_t)(n - 3 + i) * 4 * kH + row0 + t]));
            }
        }
    } else {
        __syncthreads();  // expf's table
#pragma unroll
        for (int i = 0; i < kConvR; ++i) {
            const int m = mr + MS * i;
            if (m >= nb) break;
            const size_t o = (size_t)(m0 + m) * kH + cb + c4;
            *reinterpret_cast<f32x4 *>(gate + o) = rr[i];
            *reinterpret_cast<f32x4 *>(sgate + o) =
                (f32x4){sigmoid_ref(rr[i].x, tab), sigmoid_ref(rr[i].y, tab), sigmoid_ref(rr[i].z, tab),
                        sigmoid_ref(rr[i].w, tab)};
        }
    }
}

// Per (head, token): the q/k L2 norms and alpha of the recurrence, in the
// batch-1 tree order (k_brecur's first phase), for tokens kQkTok y .. +
// kQkTok - 1 of n, their loads requested together (a token past n re-reads
// token n - 1, unused).
constexpr int kQkTok = 4;
__global__ __launch_bounds__(kT) void k_pqk(const float *__restrict__ qkv, int n, float *__restrict__ qn_out,
                                            float *__restrict__ kn_out, float *__restrict__ alpha_out) {
    static_assert(kT == kHD, "a thread per head channel");
    __shared__ float red[kQkTok][8], red2[kQkTok][4];
    const int h = blockIdx.x, m0 = (int)blockIdx.y * kQkTok, t = threadIdx.x, w = t >> 6, lane = t & 63;
    float q[kQkTok], k[kQkTok];
#pragma unroll
    for (int i = 0; i < kQkTok; ++i) {
        const float *qp = qkv + (size_t)(m0 + i < n ? m0 + i : n - 1) * 3 * kH + h * kHD;
        q[i] = qp[t];
        k[i] = qp[kH + t];
    }
#pragma unroll
    for (int i = 0; i < kQkTok; ++i) {
        const float qs = wave_tree64(q[i] * q[i]), ks = wave_tree64(k[i] * k[i]);
        if (lane == 0) {
            red[i][w] = qs;
            red[i][4 + w] = ks;
        }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kQkTok; ++i) {
        const int m = m0 + i;
        const float q_sq = (red[i][0] + red[i][1]) + (red[i][2] + red[i][3]);
        const float k_sq = (red[i][4] + red[i][5]) + (red[i][6] + red[i][7]);
        const float qv = q[i] * (1.0f / __builtin_sqrtf(q_sq + 1e-6f));
        const float kv = k[i] * (1.0f / __builtin_sqrtf(k_sq + 1e-6f));
        if (m < n) {
            qn_out[(size_t)m * kH + h * kHD + t] = qv;
            kn_out[(size_t)m * kH + h * kHD + t] = kv;
        }
        const float qk = wave_tree64(qv * kv);
        if (lane == 0) red2[i][w] = qk;
    }
    __syncthreads();
    if (t < kQkTok && m0 + t < n) alpha_out[(m0 + t) * kNH + h] = (red2[t][0] + red2[t][1]) + (red2[t][2] + red2[t][3]);
}

// The recurrence over a segment's n_total tokens in order, chunk by chunk of
// 64, one launch per layer, one wave per pair of state columns and no
// workgroup barrier inside a chunk's token loop: grid (kHD / kScanWgCols,
// kNH), four independent waves per workgroup (one per SIMD, one workgroup
// per CU; a wave64 add holds its SIMD whatever its active lanes, so two
// chain waves on one SIMD would take turns).  The state stays in registers
// from the first chunk to the last, and the next chunk's k, q, v, beta,
// decay and alpha are loaded into registers during the current token loop.
// Lane l holds rows 4 l .. 4 l + 3 of the wave's columns c0, c0 + 1 (one
// 16-byte LDS access per chain row piece).  Per token: every lane writes its
// products S[j][c] * kn[j] and S[j][c] * qn[j] to the wave's LDS rows; lanes
// 0..3 sum the chains (r of c0, r of c0 + 1, p of c0, p of c0 + 1) in row
// order j = 0..255 (the reference's chain order, adds only); the four sums
// and the token's v, beta, decay, alpha (held in lane m) are read across
// the wave, and every lane forms delta, o and its updated elements.  Each
// chunk's normalised k and q (2 x 64 x 256 FP32) are staged in LDS once.
// Each value is formed as the decode step's k_brecur forms it.
constexpr int kScanWgCols = 8;  // 4 waves x 2 columns
__global__ __launch_bounds__(kT) void k_pscan(const float *__restrict__ qkv, const float *__restrict__ qn_seg,
                                               const float *__restrict__ kn_seg, const float *__restrict__ alpha_seg,
                                               const float *__restrict__ bd_seg, int n_total, float *__restrict__ state,
                                               float *__restrict__ attn_seg) {
    constexpr int kPad = kHD + 4;  // chain rows 16 bytes apart in bank
    constexpr int KQ = kMaxB * 2 * (kHD / 4) / kT;  // staged 16-byte pieces per thread and chunk
    __shared__ __attribute__((aligned(16))) float kqs[kMaxB][2][kHD];  // [token][k|q][row]
    __shared__ __attribute__((aligned(16))) float prod[4][4 * kPad];   // [wave][chain][row]
    const int h = blockIdx.y, t = threadIdx.x, w = t >> 6, lane = t & 63;
    const int c0 = blockIdx.x * kScanWgCols + 2 * w;
    const int chunks = (n_total + kMaxB - 1) / kMaxB;
    auto chunk_len = [&](int c) { return n_total - kMaxB * c < kMaxB ? n_total - kMaxB * c : kMaxB; };
    // chunk c's normalised k and q (piece i = t + kT j: token, k|q, 4-row
    // group) and, in lane m, token m's v of both columns, beta, decay and
    // alpha: loaded into registers a chunk ahead
    f32x4 kq[KQ];
    float v0 = 0.0f, v1 = 0.0f, beta_l = 0.0f, decay_l = 0.0f, alpha_l = 0.0f;
    auto load_chunk = [&](int c) __attribute__((always_inline)) {
        const int n = chunk_len(c);
        const size_t mb = (size_t)c * kMaxB;
#pragma unroll
        for (int j = 0; j < KQ; ++j) {
            const int i = t + kT * j, m = i / (2 * (kHD / 4)), rest = i - m * 2 * (kHD / 4),
                      kind = rest / (kHD / 4), r4 = rest - kind * (kHD / 4);
            const float *src = (kind == 0 ? kn_seg : qn_seg) + (mb + m) * kH + h * kHD + 4 * r4;
            kq[j] = m < n ? *reinterpret_cast<const f32x4 *>(src) : (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
        }
        if (lane < n) {
            const float *vp = qkv + ((mb + lane) * 3 + 2) * kH + h * kHD + c0;
            v0 = vp[0];
            v1 = vp[1];
            beta_l = bd_seg[(mb + lane) * 16 + 2 * h];
            decay_l = bd_seg[(mb + lane) * 16 + 2 * h + 1];
            alpha_l = alpha_seg[(mb + lane) * kNH + h];
        }
    };
    float *S = state + (size_t)h * kHD * kHD + c0;
    float sv[2][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float2 s2 = *reinterpret_cast<const float2 *>(S + (size_t)(4 * lane + i) * kHD);
        sv[0][i] = s2.x;
        sv[1][i] = s2.y;
    }
    load_chunk(0);
    float *pw = prod[w];
    for (int c = 0; c < chunks; ++c) {
        const int n = chunk_len(c);
        float *attn = attn_seg + (size_t)c * kMaxB * kH;
#pragma unroll
        for (int j = 0; j < KQ; ++j) {
            const int i = t + kT * j, m = i / (2 * (kHD / 4)), rest = i - m * 2 * (kHD / 4), kind = rest / (kHD / 4),
                      r4 = rest - kind * (kHD / 4);
            *reinterpret_cast<f32x4 *>(&kqs[m][kind][4 * r4]) = kq[j];
        }
        // this chunk's per-token scalars, held through its token loop
        const float cv0 = v0, cv1 = v1, cbeta = beta_l, cdecay = decay_l, calpha = alpha_l;
        __syncthreads();
        if (c + 1 < chunks) load_chunk(c + 1);
        f32x4 k4n = *reinterpret_cast<const f32x4 *>(&kqs[0][0][4 * lane]);
        f32x4 q4n = *reinterpret_cast<const f32x4 *>(&kqs[0][1][4 * lane]);
        for (int m = 0; m < n; ++m) {
            const f32x4 k4 = k4n, q4 = q4n;
            const float kn[4] = {k4.x, k4.y, k4.z, k4.w};
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                *reinterpret_cast<f32x4 *>(pw + e * kPad + 4 * lane) =
                    (f32x4){sv[e][0] * k4.x, sv[e][1] * k4.y, sv[e][2] * k4.z, sv[e][3] * k4.w};
                *reinterpret_cast<f32x4 *>(pw + (2 + e) * kPad + 4 * lane) =
                    (f32x4){sv[e][0] * q4.x, sv[e][1] * q4.y, sv[e][2] * q4.z, sv[e][3] * q4.w};
            }
            // the wave's own LDS writes, then its reads of other lanes' rows
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            {
                // the next token's k and q, read while the chains run
                const int mn = m + 1 < n ? m + 1 : m;
                k4n = *reinterpret_cast<const f32x4 *>(&kqs[mn][0][4 * lane]);
                q4n = *reinterpret_cast<const f32x4 *>(&kqs[mn][1][4 * lane]);
            }
            float acc = 0.0f;
            if (lane < 4) {
                const f32x4 *col = reinterpret_cast<const f32x4 *>(pw + lane * kPad);
                f32x4 cur[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) cur[j] = col[j];
#pragma unroll
                for (int b = 0; b < kHD / 32; ++b) {
                    f32x4 nxt[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j) nxt[j] = (b + 1 < kHD / 32) ? col[8 * (b + 1) + j] : cur[j];
#pragma unroll
                    for (int j = 0; j < 8; ++j) acc = (((acc + cur[j].x) + cur[j].y) + cur[j].z) + cur[j].w;
                    asm volatile("" : "+v"(acc) : : "memory");
#pragma unroll
                    for (int j = 0; j < 8; ++j) cur[j] = nxt[j];
                }
            }
            const float ra = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), 0));
            const float rb = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), 1));
            const float pa = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), 2));
            const float pb = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), 3));
            const float beta = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cbeta), m));
            const float decay = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cdecay), m));
            const float alpha = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(calpha), m));
            const float va = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cv0), m));
            const float vb = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cv1), m));
            const float da = beta * (va - decay * ra);
            const float db = beta * (vb - decay * rb);
            if (lane < 2) {
                const float o = lane == 0 ? 0.0625f * (decay * pa + alpha * da) : 0.0625f * (decay * pb + alpha * db);
                attn[(size_t)m * kH + h * kHD + c0 + lane] = rne_bf16(o);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                sv[0][i] = decay * sv[0][i] + kn[i] * da;
                sv[1][i] = decay * sv[1][i] + kn[i] * db;
            }
            // the next token's products overwrite the rows the chains just read
            __builtin_amdgcn_wave_barrier();
        }
        // every wave is done with this chunk's rows before the next are stored
        __syncthreads();
    }
    float *Sw = S;
    asm volatile("" : "+v"(Sw));
#pragma unroll
    for (int i = 0; i < 4; ++i)
        *reinterpret_cast<float2 *>(Sw + (size_t)(4 * lane + i) * kHD) = make_float2(sv[0][i], sv[1][i]);
}

// ---------------------------------------------------- chunked prefill (WY form)
//
// The chunk's recurrence in the chunk-parallel form of the gated delta rule
// (chunk.py:616-686 computes the same quantities with a WY representation).
// With the state S (key row j, value column i) before the chunk, per-token
// decay a_m, cumulative log decay G_m = sum_{s<=m} log a_m (so a_{s+1} ...
// a_m = exp(G_m - G_s)), and normalised k_m, q_m:
//   L[m][s]  = beta_m exp(G_m - G_s) (k_m . k_s)      s < m
//   Mq[m][s] = exp(G_m - G_s) (q_m . k_s)             s <= m
//   delta_m  = beta_m (v_m - exp(G_m) S^T k_m) - sum_{s<m} L[m][s] delta_s,
//              i.e. delta = T b with T = (I + L)^-1 (formed per chunk by
//              k_wy_inv, chunk.py's solve of the same triangular system)
//   o_m      = (exp(G_m) S^T q_m + sum_{s<=m} Mq[m][s] delta_s) / 16
//   S'       = exp(G_{n-1}) S + sum_s exp(G_{n-1} - G_s) k_s delta_s^T
// which is the per-token recurrence of the decode step unrolled over the
// chunk (delta_m is the step's beta (v - decay S_{m-1}^T k), o_m its
// S_m^T q / 16).  The sums are associated differently from the step's
// sequential chains, so this mode matches the scan within a tolerance, not
// bit for bit; o is rounded to BF16 as the step rounds it.

// L and Mq of one head for rows 16 blockIdx.y .. +15 of chunk blockIdx.z of
// a segment of n_total tokens: grid (kNH, kMaxB / 16, chunks).
constexpr int kKp = kHD / 4 + 1;  // padded float4 stride of a staged k/q row

// The chunk's rows of one head ([token][kH] FP32, head h's 256 values),
// held in registers between the load and the store into LDS rows of stride
// kKp float4 (zeros from token n on).  The loads of every staged operand
// are issued at the kernel's start, so their latencies overlap instead of
// adding up.
struct RowStage {
    static constexpr int PER = kMaxB * (kHD / 4) / kT;
    f32x4 v[PER];
    __device__ __forceinline__ void load(const float *__restrict__ src, int h, int n) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int idx = threadIdx.x + kT * i, m = idx / (kHD / 4), j4 = idx % (kHD / 4);
            v[i] = m < n ? *reinterpret_cast<const f32x4 *>(src + (size_t)m * kH + h * kHD + 4 * j4)
                         : (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
        }
    }
    __device__ __forceinline__ void store(f32x4 (*rows)[kKp]) const {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int idx = threadIdx.x + kT * i;
            rows[idx / (kHD / 4)][idx % (kHD / 4)] = v[i];
        }
    }
};

// One head's 64 x 64 matrix, stored into LDS rows of stride kMaxB + 4.
struct MatStage {
    static constexpr int PER = kMaxB * kMaxB / 4 / kT;
    f32x4 v[PER];
    __device__ __forceinline__ void load(const float *__restrict__ src) {
#pragma unroll
        for (int i = 0; i < PER; ++i) v[i] = reinterpret_cast<const f32x4 *>(src)[threadIdx.x + kT * i];
    }
    __device__ __forceinline__ void store(float (*dst)[kMaxB + 4]) const {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int q = threadIdx.x + kT * i;
            *reinterpret_cast<f32x4 *>(&dst[q / (kMaxB / 4)][4 * (q % (kMaxB / 4))]) = v[i];
        }
    }
};
__device__ __forceinline__ float cum_log_decay(const float *__restrict__ bd, int h, int n, float *glog) {
    // lanes 0..63 of wave 0: inclusive prefix sum of log(decay) over the chunk
    const int lane = threadIdx.x;
    // (a decay that underflowed to 0 is taken as 1e-30: the products it
    // enters are 0 to FP32 either way, and G stays finite)
    float v = lane < n ? __logf(fmaxf(bd[lane * 16 + 2 * h + 1], 1e-30f)) : 0.0f;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const float o = __shfl_up(v, d);
        if (lane >= d) v += o;
    }
    glog[lane] = v;
    return v;
}

__global__ __launch_bounds__(kT) void k_wy_gram(const float *__restrict__ qn_seg, const float *__restrict__ kn_seg,
                                                const float *__restrict__ bd_seg, int n_total,
                                                float *__restrict__ L_seg, float *__restrict__ M_seg) {
    const int ch = blockIdx.z, n = n_total - kMaxB * ch < kMaxB ? n_total - kMaxB * ch : kMaxB;
    const float *qn_all = qn_seg + (size_t)ch * kMaxB * kH, *kn_all = kn_seg + (size_t)ch * kMaxB * kH;
    const float *bd = bd_seg + (size_t)ch * kMaxB * 16;
    float *Lout = L_seg + (size_t)ch * kNH * kMaxB * kMaxB, *Mout = M_seg + (size_t)ch * kNH * kMaxB * kMaxB;
    __shared__ f32x4 ks[kMaxB][kKp];
    __shared__ f32x4 qr[16][kKp];
    __shared__ float glog[kMaxB];
    const int h = blockIdx.x, r0 = 16 * blockIdx.y, t = threadIdx.x, w = t >> 6, lane = t & 63;
    const int li = lane & 15, kk = lane >> 4;
    RowStage kst;
    kst.load(kn_all, h, n);
    {
        // this block's 16 q rows (zeros from token n on)
        constexpr int PER = 16 * (kHD / 4) / kT;
        f32x4 v[PER];
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int idx = t + kT * i, r = idx / (kHD / 4), j4 = idx % (kHD / 4);
            v[i] = (r0 + r < n) ? *reinterpret_cast<const f32x4 *>(qn_all + (size_t)(r0 + r) * kH + h * kHD + 4 * j4)
                                : (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int idx = t + kT * i;
            qr[idx / (kHD / 4)][idx % (kHD / 4)] = v[i];
        }
    }
    kst.store(ks);
    if (t < 64) cum_log_decay(bd, h, n, glog);
    __syncthreads();
    // wave w: columns s = 16 w .. +15 of rows r0 .. r0 + 15: K_m . K_s and
    // Q_m . K_s on v_mfma_f32_16x16x4_f32 (component q of a lane's 16-byte
    // read feeds the q-th MFMA of its group, for A and B alike)
    f32x4 kk0 = {0.0f, 0.0f, 0.0f, 0.0f}, kk1 = kk0, qk0 = kk0, qk1 = kk0;
#pragma unroll
    for (int g = 0; g < kHD / 16; ++g) {
        const f32x4 ka = ks[r0 + li][4 * g + kk];
        const f32x4 qa = qr[li][4 * g + kk];
        const f32x4 kb = ks[16 * w + li][4 * g + kk];
        kk0 = __builtin_amdgcn_mfma_f32_16x16x4f32(ka.x, kb.x, kk0, 0, 0, 0);
        qk0 = __builtin_amdgcn_mfma_f32_16x16x4f32(qa.x, kb.x, qk0, 0, 0, 0);
        kk1 = __builtin_amdgcn_mfma_f32_16x16x4f32(ka.y, kb.y, kk1, 0, 0, 0);
        qk1 = __builtin_amdgcn_mfma_f32_16x16x4f32(qa.y, kb.y, qk1, 0, 0, 0);
        kk0 = __builtin_amdgcn_mfma_f32_16x16x4f32(ka.z, kb.z, kk0, 0, 0, 0);
        qk0 = __builtin_amdgcn_mfma_f32_16x16x4f32(qa.z, kb.z, qk0, 0, 0, 0);
        kk1 = __builtin_amdgcn_mfma_f32_16x16x4f32(ka.w, kb.w, kk1, 0, 0, 0);
        qk1 = __builtin_amdgcn_mfma_f32_16x16x4f32(qa.w, kb.w, qk1, 0, 0, 0);
    }
    const f32x4 gk4 = kk0 + kk1, gq4 = qk0 + qk1;
    const int sidx = 16 * w + li;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int m = r0 + 4 * kk + r;
        float lv = 0.0f, mv = 0.0f;
        if (m < n && sidx <= m) {
            const float ratio = __expf(glog[m] - glog[sidx]);
            if (sidx < m) lv = bd[m * 16 + 2 * h] * ratio * gk4[r];
            mv = ratio * gq4[r];
        }
        Lout[((size_t)h * kMaxB + m) * kMaxB + sidx] = lv;
        Mout[((size_t)h * kMaxB + m) * kMaxB + sidx] = mv;
    }
}

// T = (I + L)^-1 of one (head, chunk), in place of L: grid (kNH, chunks),
// one wave.  Lane j forms column j by forward substitution in row order,
// T[m][j] = [m == j] - sum_{s<m} L[m][s] T[s][j] (s ascending), so the
// chunk's deltas (I + L) delta = b become one matrix product, delta = T b,
// off the sequential path.  Rows of L from the chunk's length on are zero,
// so T is the identity there.
__global__ __launch_bounds__(64) void k_wy_inv(float *__restrict__ L_seg) {
    __shared__ __attribute__((aligned(16))) float ls[kMaxB][kMaxB];
    const int h = blockIdx.x, ch = blockIdx.y, j = threadIdx.x;
    float *lp = L_seg + ((size_t)ch * kNH + h) * kMaxB * kMaxB;
#pragma unroll 8
    for (int m = 0; m < kMaxB; ++m) ls[m][j] = lp[m * kMaxB + j];
    __syncthreads();
    // every row runs over all 64 columns (constant bounds, so the column
    // stays in registers): L[m][s] is exactly zero for s >= m and tc[s] is
    // still zero there, so those terms add exact zeros after the real ones
    float tc[kMaxB];
#pragma unroll
    for (int m = 0; m < kMaxB; ++m) tc[m] = 0.0f;
#pragma unroll
    for (int m = 0; m < kMaxB; ++m) {
        float acc = m == j ? 1.0f : 0.0f;
#pragma unroll
        for (int s4 = 0; s4 < kMaxB; s4 += 4) {
            const f32x4 lv = *reinterpret_cast<const f32x4 *>(&ls[m][s4]);
            acc = __builtin_fmaf(-lv.x, tc[s4], acc);
            acc = __builtin_fmaf(-lv.y, tc[s4 + 1], acc);
            acc = __builtin_fmaf(-lv.z, tc[s4 + 2], acc);
            acc = __builtin_fmaf(-lv.w, tc[s4 + 3], acc);
        }
        tc[m] = acc;
    }
#pragma unroll
    for (int m = 0; m < kMaxB; ++m) lp[m * kMaxB + j] = tc[m];
}

// One head's recurrence over a segment's chunks for 16 state columns: grid
// (kHD / kWyCols, kNH), 256 threads, the state tile held in LDS from the
// first chunk to the last and each chunk's operands loaded into registers
// while the previous chunk computes.  The matrix products run on
// v_mfma_f32_16x16x4_f32 (FP32 operands and sums; this form is held to a
// tolerance, not to the step's rounding): Q S and K S (wave w: rows 16 w ..
// +15 of the chunk, all 256 keys), the deltas T b and o (wave w: rows 16 w
// .. +15) and the state update (wave w: state rows 64 w .. +63).  An MFMA takes A[i][k] from lane i + 16 k and
// B[k][j] from lane j + 16 k and leaves D[4 (l / 16) + r][l % 16] in
// component r of lane l.  A lane reads 4 consecutive k values of its row
// (or column) in one 16-byte LDS read and feeds them to 4 MFMAs, component
// q to the q-th, so MFMA q of a group sums the k = 4 (4 g + kk) + q; A and B
// use the same assignment.
constexpr int kWyCols = 16;
constexpr int kS0p = kHD + 4;    // padded key stride of the transposed state tile
constexpr int kDtp = kMaxB + 4;  // padded token stride of the transposed deltas

__global__ __launch_bounds__(kT) void k_wy_seq(const float *__restrict__ qkv, const float *__restrict__ qn_seg,
                                               const float *__restrict__ kn_seg, const float *__restrict__ bd_seg,
                                               const float *__restrict__ T_seg, const float *__restrict__ M_seg,
                                               int n_total, float *__restrict__ state, float *__restrict__ attn) {
    __shared__ f32x4 rows[kMaxB][kKp];                                   // Q, then K
    __shared__ __attribute__((aligned(16))) float s0t[kWyCols][kS0p];    // state tile, [column][key]
    __shared__ __attribute__((aligned(16))) float lm[kMaxB][kMaxB + 4];  // T, then Mq
    __shared__ float qs[kMaxB][kWyCols + 1];                             // S^T q
    __shared__ __attribute__((aligned(16))) float bt[kWyCols][kDtp];     // b, [column][token]
    __shared__ __attribute__((aligned(16))) float dlt[kWyCols][kDtp];    // delta, [column][token]
    __shared__ __attribute__((aligned(16))) float dft[kWyCols][kDtp];    // exp(G_{n-1} - G_s) delta_s
    __shared__ float glog[kMaxB], fdec[kMaxB];
    const int h = blockIdx.y, c0 = blockIdx.x * kWyCols, t = threadIdx.x, w = t >> 6, lane = t & 63;
    const int li = lane & 15, kk = lane >> 4;  // MFMA operand row/column, k quarter
    const int chunks = (n_total + kMaxB - 1) / kMaxB;
    const size_t mat = (size_t)kNH * kMaxB * kMaxB;  // one chunk's L (or Mq), every head
    float *S = state + (size_t)h * kHD * kHD + c0;
    auto chunk_len = [&](int c) { return n_total - kMaxB * c < kMaxB ? n_total - kMaxB * c : kMaxB; };
    // the operands of chunk c into registers (issued a chunk ahead)
    RowStage qst, kst;
    MatStage lst, mst;
    float vv[4], beta[4], dec = 1.0f;
    auto load_vb = [&](int c) __attribute__((always_inline)) {
        const int n = chunk_len(c);
        const size_t m0 = (size_t)c * kMaxB;
        // v and beta of this lane's D elements of K S: rows 16 w + 4 kk + r, column li
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = 16 * w + 4 * kk + r;
            vv[r] = m < n ? qkv[((m0 + m) * 3 + 2) * kH + h * kHD + c0 + li] : 0.0f;
            beta[r] = m < n ? bd_seg[(m0 + m) * 16 + 2 * h] : 0.0f;
        }
        dec = lane < n ? bd_seg[(m0 + lane) * 16 + 2 * h + 1] : 1.0f;
    };
    qst.load(qn_seg, h, chunk_len(0));
    lst.load(T_seg + (size_t)h * kMaxB * kMaxB);
    kst.load(kn_seg, h, chunk_len(0));
    mst.load(M_seg + (size_t)h * kMaxB * kMaxB);
    load_vb(0);
    {
        const f32x4 *src = reinterpret_cast<const f32x4 *>(S + (size_t)t * kHD);
        f32x4 v[kWyCols / 4];
#pragma unroll
        for (int i = 0; i < kWyCols / 4; ++i) v[i] = src[i];
#pragma unroll
        for (int i = 0; i < kWyCols / 4; ++i) {
            s0t[4 * i][t] = v[i].x;
            s0t[4 * i + 1][t] = v[i].y;
            s0t[4 * i + 2][t] = v[i].z;
            s0t[4 * i + 3][t] = v[i].w;
        }
    }

    // X S for the staged rows X (Q, then K): rows 16 w .. +15, 256 keys
    const auto xs_mfma = [&]() __attribute__((always_inline)) {
        f32x4 acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = acc0;
#pragma unroll
        for (int g = 0; g < kHD / 16; ++g) {
            const f32x4 xa = rows[16 * w + li][4 * g + kk];
            const f32x4 xb = *reinterpret_cast<const f32x4 *>(&s0t[li][16 * g + 4 * kk]);
            acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(xa.x, xb.x, acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(xa.y, xb.y, acc1, 0, 0, 0);
            acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(xa.z, xb.z, acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(xa.w, xb.w, acc1, 0, 0, 0);
        }
        return acc0 + acc1;
    };

    for (int c = 0; c < chunks; ++c) {
        const int n = chunk_len(c);
        const bool more = c + 1 < chunks;
        const size_t m0 = (size_t)c * kMaxB, m1 = m0 + kMaxB;
        qst.store(rows);
        lst.store(lm);
        if (more) {
            qst.load(qn_seg + m1 * kH, h, chunk_len(c + 1));
            lst.load(T_seg + (c + 1) * mat + (size_t)h * kMaxB * kMaxB);
        }
        if (t < 64) {
            // inclusive prefix sum of log(decay) over the chunk (a decay that
            // underflowed to 0 is taken as 1e-30: the products it enters are 0
            // to FP32 either way, and G stays finite)
            float v = lane < n ? __logf(fmaxf(dec, 1e-30f)) : 0.0f;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const float o = __shfl_up(v, d);
                if (lane >= d) v += o;
            }
            glog[lane] = v;
        }
        __syncthreads();
        if (t < kMaxB) fdec[t] = __expf(glog[n - 1] - glog[t]);

        // S^T q for every token
        {
            const f32x4 d = xs_mfma();
#pragma unroll
            for (int r = 0; r < 4; ++r) qs[16 * w + 4 * kk + r][li] = d[r];
        }
        __syncthreads();
        kst.store(rows);
        if (more) kst.load(kn_seg + m1 * kH, h, chunk_len(c + 1));
        __syncthreads();
        // S^T k for every token, then b_m = beta_m (v_m - exp(G_m) S^T k_m)
        {
            const f32x4 d = xs_mfma();
            f32x4 b;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = 16 * w + 4 * kk + r;
                b[r] = m < n ? beta[r] * (vv[r] - __expf(glog[m]) * d[r]) : 0.0f;
            }
            *reinterpret_cast<f32x4 *>(&bt[li][16 * w + 4 * kk]) = b;
        }
        __syncthreads();
        if (more) load_vb(c + 1);

        // delta = T b: rows 16 w .. +15 (zero from row n on, where b is
        // zero and T the identity), transposed for the MFMA B operands and
        // scaled by their decay for the state update
        {
            f32x4 acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = acc0;
#pragma unroll
            for (int g = 0; g < kMaxB / 16; ++g) {
                const f32x4 xa = *reinterpret_cast<const f32x4 *>(&lm[16 * w + li][16 * g + 4 * kk]);
                const f32x4 xb = *reinterpret_cast<const f32x4 *>(&bt[li][16 * g + 4 * kk]);
                acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(xa.x, xb.x, acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(xa.y, xb.y, acc1, 0, 0, 0);
                acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(xa.z, xb.z, acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(xa.w, xb.w, acc1, 0, 0, 0);
            }
            const f32x4 d = acc0 + acc1;
            const int m = 16 * w + 4 * kk;
            *reinterpret_cast<f32x4 *>(&dlt[li][m]) = d;
            *reinterpret_cast<f32x4 *>(&dft[li][m]) =
                (f32x4){fdec[m] * d[0], fdec[m + 1] * d[1], fdec[m + 2] * d[2], fdec[m + 3] * d[3]};
        }
        __syncthreads();
        mst.store(lm);
        if (more) mst.load(M_seg + (c + 1) * mat + (size_t)h * kMaxB * kMaxB);
        __syncthreads();

        // o_m = (exp(G_m) S^T q_m + sum_{s<=m} Mq[m][s] delta_s) / 16,
        // rounded: rows 16 w .. +15
        {
            f32x4 acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = acc0;
#pragma unroll
            for (int g = 0; g < kMaxB / 16; ++g) {
                const f32x4 xa = *reinterpret_cast<const f32x4 *>(&lm[16 * w + li][16 * g + 4 * kk]);
                const f32x4 xb = *reinterpret_cast<const f32x4 *>(&dlt[li][16 * g + 4 * kk]);
                acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(xa.x, xb.x, acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(xa.y, xb.y, acc1, 0, 0, 0);
                acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(xa.z, xb.z, acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(xa.w, xb.w, acc1, 0, 0, 0);
            }
            const f32x4 d = acc0 + acc1;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = 16 * w + 4 * kk + r;
                if (m < n) {
                    const float o = __expf(glog[m]) * qs[m][li] + d[r];
                    attn[(m0 + m) * kH + h * kHD + c0 + li] = rne_bf16(0.0625f * o);
                }
            }
        }

        // S' = exp(G_{n-1}) S + sum_s exp(G_{n-1} - G_s) k_s delta_s^T:
        // state rows 64 w .. +63 as four 16-row tiles; A[j][s] = k_s[j]
        // (token rows of the staged K), B[s][c] = exp(G_{n-1} - G_s)
        // delta_s[c].  Each element is read and rewritten in place by the
        // lane that owns it.
        {
            const float dn = __expf(glog[n - 1]);
            const float *krow = reinterpret_cast<const float *>(&rows[0][0]);
#pragma unroll
            for (int tile = 0; tile < 4; ++tile) {
                const int j0 = 64 * w + 16 * tile;
                f32x4 acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = acc0;
#pragma unroll
                for (int g = 0; g < kMaxB / 16; ++g) {
                    const int sb = 16 * g + 4 * kk;  // this lane's 4 tokens
                    const f32x4 xb = *reinterpret_cast<const f32x4 *>(&dft[li][sb]);
                    const float a0 = krow[(sb + 0) * (4 * kKp) + j0 + li];
                    const float a1 = krow[(sb + 1) * (4 * kKp) + j0 + li];
                    const float a2 = krow[(sb + 2) * (4 * kKp) + j0 + li];
                    const float a3 = krow[(sb + 3) * (4 * kKp) + j0 + li];
                    acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, xb.x, acc0, 0, 0, 0);
                    acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, xb.y, acc1, 0, 0, 0);
                    acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(a2, xb.z, acc0, 0, 0, 0);
                    acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(a3, xb.w, acc1, 0, 0, 0);
                }
                const f32x4 d = acc0 + acc1;
                f32x4 *sp = reinterpret_cast<f32x4 *>(&s0t[li][j0 + 4 * kk]);
                const f32x4 sv = *sp;
                *sp = (f32x4){__builtin_fmaf(dn, sv[0], d[0]), __builtin_fmaf(dn, sv[1], d[1]),
                              __builtin_fmaf(dn, sv[2], d[2]), __builtin_fmaf(dn, sv[3], d[3])};
            }
        }
        // the next chunk overwrites rows, lm and the deltas
        __syncthreads();
    }
    {
        f32x4 *dst = reinterpret_cast<f32x4 *>(S + (size_t)t * kHD);
#pragma unroll
        for (int i = 0; i < kWyCols / 4; ++i)
            dst[i] = (f32x4){s0t[4 * i][t], s0t[4 * i + 1][t], s0t[4 * i + 2][t], s0t[4 * i + 3][t]};
    }
}

// ------------------------------------------------ prefill projections
//
// A prefill segment runs layer by layer, so each layer's projection weights
// are read once per segment instead of once per 64 tokens.  k_pgemm (and
// k_pgemm_a, below) and k_pgu form the segment's projections as GEMMs: one workgroup per 128 rows
// (four 32-row blocks of the weight layout; gate/up: two channel groups) x
// 128 tokens (two 64-token X tile blocks), eight waves of 64 rows x 32
// tokens, the k tile's fragments staged once through LDS (double buffer,
// two k tiles of loads in flight per thread).  Every output element is
// formed with the step's operations in the step's order: the same
// v_mfma_f32_16x16x32_bf16 fragments; the k tiles of class c (c, c + NW,
// ... within a split) chained from zero in increasing order, as wave c of
// k_bgemm / k_bgu chains them; the classes added in order, as k_bgemm adds
// its waves' sums; and the splits' sums added in split order, as the
// step's norm adds k_bgemm's split partials.  A prefill therefore still
// equals the steps bit for bit.
#ifndef GDN_PG_DEPTH
#define GDN_PG_DEPTH 2
#endif
constexpr int kPgD = GDN_PG_DEPTH;  // k tiles of operand loads in flight per thread
constexpr int kPgTok = 128;  // tokens per workgroup (2 X tile blocks)
constexpr int kSegDefault = 4096;  // prefill tokens per segment by default
constexpr int kSegMax = 32768;     // largest segment (k_pqk's grid.y holds it)

// The j-th k tile in class order: split s, class c, i-th tile of the class.
template <int KT, int NW, int S>
__device__ __forceinline__ int pg_tile(int j) {
    constexpr int KTS = KT / S, KTW = KTS / NW;
    const int s = j / KTS, r = j - s * KTS, c = r / KTW, i = r - c * KTW;
    return s * KTS + c + NW * i;
}

// The workgroup's (row tile, token tile).  Workgroups are dealt to the 8
// XCDs round robin in launch order; when the grid allows, the 32 that one
// XCD runs together cover 4 row tiles x 8 token tiles (a "super tile"), so
// that XCD's L2 serves each weight tile to 8 of them and each activation
// tile to 4.  Otherwise the plain (blockIdx.x, blockIdx.y).
__device__ __forceinline__ void pg_place(int &rt, int &tt) {
    const int R = gridDim.x, C = gridDim.y, L = blockIdx.x + R * blockIdx.y;
    if (R % 4 == 0 && C % 8 == 0 && (R * C) % 256 == 0) {
        const int x = L & 7, s = L >> 3;
        const int u = 8 * (s >> 5) + x, q = s & 31, gr = R / 4;
        rt = 4 * (u % gr) + (q & 3);
        tt = 8 * (u / gr) + (q >> 2);
    } else {
        rt = blockIdx.x;
        tt = blockIdx.y;
    }
}

// Class bookkeeping after k tile j: the class chain joins the split's sum
// (the first class is taken as it is).  Returns true when the tile closes a
// split (its sum is complete in part).
template <int KT, int NW, int S, int NB>
__device__ __forceinline__ bool pg_close(int j, f32x4 (&chain)[NB], f32x4 (&part)[NB]) {
    constexpr int KTS = KT / S, KTW = KTS / NW;
    if ((j + 1) % KTW != 0) return false;
    const int cls = ((j + 1) / KTW - 1) % NW;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        part[b] = cls == 0 ? chain[b] : part[b] + chain[b];
        chain[b] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    }
    return cls == NW - 1;
}

// y[m][row] for rows 128 rt .. +127 and tokens 128 tt .. +127 (pg_place):
// the sum k_bgemm<2, KT, NW, S, EPI_RAW> forms for the row (S = 1), or the
// in-order sum of its S split partials.  With splits the running total
// lives in the output tile itself (each lane rewrites only its own
// elements, after its own earlier store), so a wave holds only two
// accumulator sets (the class chain and the split's sum).  W in the 32-row
// block layout ([row block][k tile][2 tiles][64 lanes]); X in 64-token X
// tile blocks; y has the padded token count's rows.
// Waves per workgroup: 8 of 64 rows x 32 tokens (about 100 VGPRs, four
// waves per SIMD) measured 98.4k against 95.9k prefill tokens/s for 4 of
// 64 x 64 (two per SIMD), with twice the LDS fragment reads.
#ifndef GDN_PG_WAVES
#define GDN_PG_WAVES 8
#endif
constexpr int kPgW = GDN_PG_WAVES;

template <int KT, int NW, int S>
__global__ __launch_bounds__(kPgW * 64) void k_pgemm(const u32x4 *__restrict__ W, const u32x4 *__restrict__ X,
                                                     float *__restrict__ y, int n_rows) {
    constexpr int GT = kPgW * 64, AU = 4 * 2 * 64, BU = 2 * 4 * 64, PT = (AU + BU) / GT;
    constexpr int TG = kPgW == 4 ? 4 : 2;  // 16-token groups per wave
    constexpr int NB = 4 * TG;            // 16 x 16 blocks per wave
    static_assert(kPgW == 4 || kPgW == 8, "four or eight waves");
    static_assert(KT % kPgD == 0 && kPgD % 2 == 0, "whole groups of kPgD k tiles");
    __shared__ u32x4 stg[2][AU + BU];
    const int t = threadIdx.x, w = t >> 6, l = t & 63, wr = w & 1, wt = w >> 1;
    int rt, tt;
    pg_place(rt, tt);
    // entry q = t + GT i: A (row block q / 128, entry q % 128) below AU,
    // else B (token block, entry)
    const u32x4 *src[PT];
    int stride[PT];
#pragma unroll
    for (int i = 0; i < PT; ++i) {
        const int q = t + GT * i;
        if (q < AU) {
            src[i] = W + (size_t)(4 * rt + q / 128) * KT * 128 + (q % 128);
            stride[i] = 128;
        } else {
            src[i] = X + (size_t)(2 * tt + (q - AU) / 256) * KT * 256 + ((q - AU) % 256);
            stride[i] = 256;
        }
    }
    auto fetch = [&](u32x4 (&r)[PT], int kt) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < PT; ++i) r[i] = src[i][(size_t)kt * stride[i]];
    };
    f32x4 chain[NB], part[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) chain[b] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    // row tile f: rows 128 rt + 64 wr + 16 f + 4 (l / 16) .. +3; token
    // group g of the wave: token 128 tt + 16 (TG wt + g) + l % 16
    const int row = 128 * rt + 64 * wr + 4 * (l >> 4);
    const int m = kPgTok * tt + 16 * TG * wt + (l & 15);
    auto out = [&](int b) {
        return reinterpret_cast<f32x4 *>(y + (size_t)(m + 16 * (b % TG)) * n_rows + row + 16 * (b / TG));
    };
    u32x4 rg[kPgD][PT];
#pragma unroll
    for (int d = 0; d < kPgD; ++d) fetch(rg[d], pg_tile<KT, NW, S>(d));
    for (int j0 = 0; j0 < KT; j0 += kPgD) {
#pragma unroll
        for (int d = 0; d < kPgD; ++d) {
            const int j = j0 + d, sb = d & 1;
#pragma unroll
            for (int i = 0; i < PT; ++i) stg[sb][t + GT * i] = rg[d][i];
            // issued on every pass (the last passes re-read the final tile,
            // unused): a conditional load would make the compiler's wait
            // for the next stage a wait for every load in flight
            fetch(rg[d], pg_tile<KT, NW, S>(j + kPgD < KT ? j + kPgD : KT - 1));
            __syncthreads();
            u32x4 fa[4], fb[TG];
#pragma unroll
            for (int f = 0; f < 4; ++f) fa[f] = stg[sb][256 * wr + 64 * f + l];
#pragma unroll
            for (int g = 0; g < TG; ++g) fb[g] = stg[sb][AU + 64 * (TG * wt + g) + l];
#pragma unroll
            for (int f = 0; f < 4; ++f)
#pragma unroll
                for (int g = 0; g < TG; ++g)
                    chain[TG * f + g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        __builtin_bit_cast(bf16x8, fa[f]), __builtin_bit_cast(bf16x8, fb[g]), chain[TG * f + g], 0,
                        0, 0);
            if (pg_close<KT, NW, S, NB>(j, chain, part)) {
                // the split's sum joins the total in split order
                const bool first = j < KT / S;
#pragma unroll
                for (int b = 0; b < NB; ++b) *out(b) = first ? part[b] : *out(b) + part[b];
            }
        }
    }
}

// k_pgemm with the weights streamed straight into registers: one workgroup
// per 32 kPgW rows (a 32-row block per wave) x 128 tokens, wave w owning
// rows 32 w .. 32 w + 31 of them for all 128 tokens, so no two waves need the same
// weight fragment and only the tokens' fragments (8 KB per k tile) pass
// through LDS.  The k loop runs one class of one split per trip (its KTW
// tiles unrolled, the next kPaD tiles' operands in flight across trips):
// a loop of fixed shape, whose waits on memory the compiler keeps exact,
// where a loop of kPgD tiles with a data-dependent class close waited for
// every load in flight at its top.  Same fragments, chains, class order and
// split order as k_pgemm, so the same sums bit for bit.  Traced in the
// 4096-token prefill: q/k/v/g 169.5 -> 150.0 us, down 138.9 -> 127.9 us.
// o_proj (16 k tiles per split) stays on k_pgemm, as it measured no faster
// in isolation; so does any launch whose grid would not fill the CUs
// (pa_fills), where k_pgemm's twice as many workgroups do better.
constexpr int kPaRows = 32 * kPgW;  // rows per workgroup
constexpr int kPaD = 2;       // k tiles of operands in flight
template <int KT, int NW, int S>
__global__ __launch_bounds__(kPgW * 64) void k_pgemm_a(const u32x4 *__restrict__ W, const u32x4 *__restrict__ X,
                                                       float *__restrict__ y, int n_rows) {
    constexpr int R = kPaRows / 16 / kPgW;  // 16-row tiles per wave
    constexpr int T = kPgTok / 16;          // 16-token groups per wave
    constexpr int GT = kPgW * 64, BU = T * 64, PB = BU / GT;
    constexpr int NB = R * T, KTS = KT / S, KTW = KTS / NW;
    static_assert(R == 2 && BU % GT == 0 && KT % S == 0 && KTS % NW == 0, "row and token tiles per workgroup");
    __shared__ u32x4 stg[2][BU];
    const int t = threadIdx.x, w = t >> 6, l = t & 63;
    int rt, tt;
    pg_place(rt, tt);
    // wave w's rows: 32-row block kPgW rt + w of the weight layout (its two
    // tiles at entries 0..63 and 64..127 of each k tile)
    const u32x4 *ap = W + (size_t)(kPgW * rt + w) * KT * 128 + l;
    // B entry q of a k tile: token group q / 64 (of 8), lane q % 64
    const u32x4 *bp[PB];
#pragma unroll
    for (int i = 0; i < PB; ++i) {
        const int q = t + GT * i;
        bp[i] = X + (size_t)(2 * tt + (q >> 8)) * KT * 256 + (q & 255);
    }
    f32x4 chain[NB], part[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        chain[b] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
        part[b] = chain[b];
    }
    u32x4 ra[kPaD][R], rb[kPaD][PB];
#pragma unroll
    for (int d = 0; d < kPaD; ++d) {
        const int kt = pg_tile<KT, NW, S>(d);
#pragma unroll
        for (int f = 0; f < R; ++f) ra[d][f] = ap[(size_t)kt * 128 + 64 * f];
#pragma unroll
        for (int i = 0; i < PB; ++i) rb[d][i] = bp[i][(size_t)kt * 256];
    }
    // row tile f: rows kPaRows rt + 32 w + 16 f + 4 (l / 16) .. +3; token group
    // g: token 128 tt + 16 g + l % 16
    const int row = kPaRows * rt + 32 * w + 4 * (l >> 4);
    const int m = kPgTok * tt + (l & 15);
    auto out = [&](int f, int g) {
        return reinterpret_cast<f32x4 *>(y + (size_t)(m + 16 * g) * n_rows + row + 16 * f);
    };
    for (int c = 0; c < KT / KTW; ++c) {
#pragma unroll
        for (int i = 0; i < KTW; ++i) {
            const int j = c * KTW + i, sb = j & 1;
            u32x4 fa[R];
#pragma unroll
            for (int f = 0; f < R; ++f) fa[f] = ra[0][f];
#pragma unroll
            for (int q = 0; q < PB; ++q) stg[sb][t + GT * q] = rb[0][q];
#pragma unroll
            for (int d = 0; d + 1 < kPaD; ++d) {
#pragma unroll
                for (int f = 0; f < R; ++f) ra[d][f] = ra[d + 1][f];
#pragma unroll
                for (int q = 0; q < PB; ++q) rb[d][q] = rb[d + 1][q];
            }
            {
                // issued on every tile (the last ones re-read the final tile,
                // unused), so the loop's shape stays fixed
                const int kt = pg_tile<KT, NW, S>(j + kPaD < KT ? j + kPaD : KT - 1);
#pragma unroll
                for (int f = 0; f < R; ++f) ra[kPaD - 1][f] = ap[(size_t)kt * 128 + 64 * f];
#pragma unroll
                for (int q = 0; q < PB; ++q) rb[kPaD - 1][q] = bp[q][(size_t)kt * 256];
            }
            __syncthreads();
            u32x4 fb[T];
#pragma unroll
            for (int g = 0; g < T; ++g) fb[g] = stg[sb][64 * g + l];
#pragma unroll
            for (int g = 0; g < T; ++g)
#pragma unroll
                for (int f = 0; f < R; ++f)
                    chain[T * f + g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        __builtin_bit_cast(bf16x8, fa[f]), __builtin_bit_cast(bf16x8, fb[g]), chain[T * f + g], 0, 0,
                        0);
        }
        // class c % NW of split c / NW closes: its chain joins the split's
        // sum, and the last class's sum joins the total in split order
        const int cls = c % NW;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            part[b] = cls == 0 ? chain[b] : part[b] + chain[b];
            chain[b] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
        }
        if (cls == NW - 1) {
            const bool first = c < NW;
#pragma unroll
            for (int f = 0; f < R; ++f)
#pragma unroll
                for (int g = 0; g < T; ++g) *out(f, g) = first ? part[T * f + g] : *out(f, g) + part[T * f + g];
        }
    }
}

// Gate/up + SwiGLU for channel groups 2 rt, +1 (k_bgu's layout and sums:
// four classes of 16 k tiles) and tokens 128 tt .. +127 (pg_place; the
// first n_tok are written).  Wave w: group w & 1, token block w >> 1.
__global__ __launch_bounds__(kPgW * 64) void k_pgu(const u32x4 *__restrict__ W, const u32x4 *__restrict__ X,
                                                   uint16_t *__restrict__ x_next, int n_tok) {
    constexpr int KT = kKtH, NW = kGuWaves, GT = kPgW * 64;
    constexpr int AU = 2 * kGuTileU4, BU = 2 * 4 * 64, PT = (AU + BU + GT - 1) / GT;
    constexpr int TG = kPgW == 4 ? 4 : 2;  // 16-token groups per wave
    constexpr int NB = 3 * TG;            // 16 x 16 blocks per wave
    static_assert(kPgW == 4 || kPgW == 8, "four or eight waves");
    static_assert(KT % kPgD == 0 && kPgD % 2 == 0, "whole groups of kPgD k tiles");
    __shared__ u32x4 stg[2][AU + BU];
    __shared__ f32x4 red[kPgW][NB * 64];
    __shared__ uint64_t exp2_lds[32];  // expf's table for the SwiGLU epilogue
    const int t = threadIdx.x, w = t >> 6, l = t & 63, wg = w & 1, wt = w >> 1;
    int rt, tt;
    pg_place(rt, tt);
    const int gb = 2 * rt;
    fill_exp2_lds_imm(exp2_lds);
    // entry q = t + GT i: A (group q / kGuTileU4) below AU, else B
    const u32x4 *src[PT];
    int stride[PT];
    bool live[PT];
#pragma unroll
    for (int i = 0; i < PT; ++i) {
        const int q = t + GT * i;
        live[i] = q < AU + BU;
        // entries past the end re-read B entry 0 (loaded, not stored), so
        // every load is unconditional
        if (q < AU) {
            src[i] = W + (size_t)(gb + q / kGuTileU4) * KT * kGuTileU4 + (q % kGuTileU4);
            stride[i] = kGuTileU4;
        } else {
            const int qb = live[i] ? q - AU : 0;
            src[i] = X + (size_t)(2 * tt + qb / 256) * KT * 256 + (qb % 256);
            stride[i] = 256;
        }
    }
    auto fetch = [&](u32x4 (&r)[PT], int kt) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < PT; ++i) r[i] = src[i][(size_t)kt * stride[i]];
    };
    const bool p2 = (l & 15) < kGuTail2;
    const int o2 = 128 + (p2 ? (l >> 4) * kGuTail2 + (l & 15) : 0);
    const u32x4 zero = {0u, 0u, 0u, 0u};
    f32x4 chain[NB], part[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) chain[b] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    u32x4 rg[kPgD][PT];
#pragma unroll
    for (int d = 0; d < kPgD; ++d) fetch(rg[d], pg_tile<KT, NW, 1>(d));
    for (int j0 = 0; j0 < KT; j0 += kPgD) {
#pragma unroll
        for (int d = 0; d < kPgD; ++d) {
            const int j = j0 + d, sb = d & 1;
#pragma unroll
            for (int i = 0; i < PT; ++i)
                if (live[i]) stg[sb][t + GT * i] = rg[d][i];
            fetch(rg[d], pg_tile<KT, NW, 1>(j + kPgD < KT ? j + kPgD : KT - 1));
            __syncthreads();
            u32x4 fa[3], fb[TG];
            fa[0] = stg[sb][wg * kGuTileU4 + l];
            fa[1] = stg[sb][wg * kGuTileU4 + 64 + l];
            fa[2] = p2 ? stg[sb][wg * kGuTileU4 + o2] : zero;
#pragma unroll
            for (int g = 0; g < TG; ++g) fb[g] = stg[sb][AU + 64 * (TG * wt + g) + l];
#pragma unroll
            for (int f = 0; f < 3; ++f)
#pragma unroll
                for (int g = 0; g < TG; ++g)
                    chain[TG * f + g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        __builtin_bit_cast(bf16x8, fa[f]), __builtin_bit_cast(bf16x8, fb[g]), chain[TG * f + g], 0,
                        0, 0);
            (void)pg_close<KT, NW, 1, NB>(j, chain, part);
        }
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) red[w][b * 64 + l] = part[b];
    // the wave reads only its own sums
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // row rr of tile r, token m of the wave: lane (rr / 4) * 16 + m % 16 of
    // token group m / 16, component rr % 4 (k_bgu's val)
    auto val = [&](int r, int rr, int m) {
        return reinterpret_cast<const float *>(red[w])[4 * ((r * TG + (m >> 4)) * 64 + (rr >> 2) * 16 + (m & 15)) +
                                                       (rr & 3)];
    };
    const int mb = kPgTok * tt + 16 * TG * wt;
    for (int q = l; q < 16 * TG * (kGuCh / 2); q += 64) {
        const int m = q / (kGuCh / 2), cp = q - m * (kGuCh / 2);
        if (mb + m >= n_tok) continue;
        uint32_t packed = 0;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int cc = 2 * cp + e;
            const float g = rne_bf16(cc < 16 ? val(0, cc, m) : val(2, cc - 16, m));
            const float u = rne_bf16(cc < 16 ? val(1, cc, m) : val(2, cc - 16 + (kGuCh - 16), m));
            packed |= bf16_daz_bits(rne_bf16(silu_ref(g, Exp2Lds{exp2_lds}) * u)) << (16 * e);
        }
        *reinterpret_cast<uint32_t *>(x_next + xt_index(mb + m, (gb + wg) * kGuCh + 2 * cp, kI)) = packed;
    }
}

}  // namespace bt
}  // namespace gdn

// ===================================================================== engine

using namespace gdn;
using namespace gdn::bt;

struct GDNBatchEngine {
    int layers = 0, vocab = 0, streams = 0;
    float eps = 1e-6f;
    hipStream_t stream = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    void *wmem = nullptr;
    const u32x4 *w_qkvg[kMaxLayers] = {}, *w_o[kMaxLayers] = {}, *w_gu[kMaxLayers] = {},
                *w_down[kMaxLayers] = {}, *w_lm = nullptr;
    uint16_t *emb = nullptr;
    float *aux = nullptr;      // [layers][kAuxLayer] + final_norm[kH]
    float *state = nullptr;    // [layers][streams][kNH][kHD][kHD]
    uint16_t *tails = nullptr; // [layers][streams][3][3][kH], BF16 bits
    float *act = nullptr;
    float *h = nullptr, *qkv = nullptr, *gate = nullptr, *sgate = nullptr, *bd = nullptr,
          *attn = nullptr, *ypart = nullptr, *xn = nullptr, *logits = nullptr, *part_val = nullptr;
    int *part_idx = nullptr;
    uint16_t *x_h = nullptr, *x_o = nullptr, *x_d = nullptr;  // X tiles, K = 2048 / 2048 / 5632
    int *tok_host = nullptr;  // pinned, mapped, coherent: [0..64) tokens in, [64..128) argmaxes out
    int *tok_map = nullptr;   // the device's address of tok_host (the step's tokens)
    // prefill: the last token block's logits and argmax tokens (buffers of
    // their own, so a prefill leaves the other streams' last step readable)
    float *p_logits = nullptr;
    int *p_tok = nullptr;
    int prefill_mode = GDN_PREFILL_SCAN;
    // prefill segment buffers, allocated at the first prefill for seg_cap
    // tokens (per token: residual ping-pong, projection sums, q/k/v, gate,
    // sigmoid(gate), beta/decay, attention output, normalised q/k, alpha,
    // the chunk matrices L and Mq, final hidden; X tiles of three widths)
    int seg_tokens = kSegDefault, seg_cap = 0;
    void *seg_mem = nullptr;
    float *s_h = nullptr, *s_y = nullptr, *s_qkv = nullptr, *s_gate = nullptr, *s_sgate = nullptr, *s_bd = nullptr,
          *s_attn = nullptr, *s_qn = nullptr, *s_kn = nullptr, *s_alpha = nullptr, *s_wyl = nullptr,
          *s_wym = nullptr, *s_xn = nullptr;
    uint16_t *s_xh = nullptr, *s_xo = nullptr, *s_xd = nullptr;
    int *s_tok = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    bool use_graph = true;
};

namespace {

float *b_aux(GDNBatchEngine *e, int l) { return e->aux + (size_t)l * kAuxLayer; }
uint16_t *b_tails(GDNBatchEngine *e, int l) { return e->tails + (size_t)l * e->streams * kStreamTails; }
float *b_state(GDNBatchEngine *e, int l) { return e->state + (size_t)l * e->streams * kLayerState; }
// The LM head takes 64 rows per workgroup (half the activation re-reads of
// 32: 35.1 -> 28.8 us for the 32000-row head, same sums) where the vocabulary
// allows, else 32; its weights are tiled to match.
int lm_rt(const GDNBatchEngine *e) { return (e->vocab % 64) == 0 ? 4 : 2; }
int lm_wgs(const GDNBatchEngine *e) { return e->vocab / (16 * lm_rt(e)); }
void launch_lm_gemm(GDNBatchEngine *e, const BEpi &ep, const void *x, hipStream_t s) {
    const u32x4 *x4 = reinterpret_cast<const u32x4 *>(x);
    if (lm_rt(e) == 4)
        hipLaunchKernelGGL((k_bgemm<4, kKtH, 4, 1, EPI_LM>), dim3(lm_wgs(e)), dim3(kT), 0, s, e->w_lm, x4, ep);
    else
        hipLaunchKernelGGL((k_bgemm<2, kKtH, 4, 1, EPI_LM>), dim3(lm_wgs(e)), dim3(kT), 0, s, e->w_lm, x4, ep);
}

int b_check_shape(const GDNWeightHeader *c) {
    if (c->hidden_size != (uint32_t)kH || c->num_heads != (uint32_t)kNH || c->num_v_heads != (uint32_t)kNH ||
        c->head_dim != (uint32_t)kHD || c->intermediate_size != (uint32_t)kI || c->conv_size != 4u) {
        gdn_error("gdn: the engine is specialised for hidden 2048, 8x256 heads, intermediate 5632, conv 4");
        return -1;
    }
    if (c->num_layers < 1 || c->num_layers > (uint32_t)kMaxLayers) {
        gdn_error("gdn: num_layers must be 1..24");
        return -1;
    }
    if (c->vocab_size == 0 || (c->vocab_size % 32) != 0) {
        gdn_error("gdn: the multi-stream engine needs a vocabulary that is a multiple of 32");
        return -1;
    }
    return 0;
}

// BF16 bits (subnormals flushed) of n BF16-exact floats.
void to_bf16(const float *src, size_t n, std::vector<uint16_t> &dst) {
    dst.resize(n);
    float mn, mx;
    int bad;
    gdn_pack_bf16_daz(src, dst.data(), n, &mn, &mx, &bad);
}

int upload_tiled(const std::vector<uint16_t> &rows, size_t n_rows, size_t k, int rt, char *&p,
                 const u32x4 *&out) {
    std::vector<uint16_t> tiled(n_rows * k);
    gdn_tile_bf16(rows.data(), n_rows, k, rt, tiled.data());
    GDN_HIP(hipMemcpy(p, tiled.data(), tiled.size() * 2, hipMemcpyHostToDevice));
    out = reinterpret_cast<const u32x4 *>(p);
    p += tiled.size() * 2;
    return 0;
}

// Gate [kI][kH] and up [kI][kH] BF16 rows in k_bgu's layout: per workgroup b
// and k tile, gate rows 22 b .. + 15 and up rows 22 b .. + 15 as A-operand
// tiles, then the 12-row tile (gate rows 22 b + 16 .. + 21, up rows likewise)
// as (quarter, row) entries.
void tile_gu(const uint16_t *g, const uint16_t *u, uint16_t *dst) {
    const size_t K = kH;
#pragma omp parallel for schedule(static)
    for (int b = 0; b < kGuWgs; ++b)
        for (int kt = 0; kt < kKtH; ++kt) {
            uint16_t *tile = dst + ((size_t)b * kKtH + kt) * kGuTileU4 * 8;
            const size_t col = (size_t)kt * 32;
            for (int l = 0; l < 64; ++l) {
                const size_t ch = (size_t)b * kGuCh + l % 16, c8 = col + 8 * (l / 16);
                std::memcpy(tile + l * 8, g + ch * K + c8, 16);
                std::memcpy(tile + (64 + l) * 8, u + ch * K + c8, 16);
            }
            constexpr int kTail = kGuCh - 16;
            for (int kq = 0; kq < 4; ++kq)
                for (int r = 0; r < kGuTail2; ++r) {
                    const size_t ch = (size_t)b * kGuCh + 16 + (r % kTail);
                    std::memcpy(tile + (128 + kq * kGuTail2 + r) * 8, (r < kTail ? g : u) + ch * K + col + 8 * kq,
                                16);
                }
        }
}

int b_upload(GDNBatchEngine *e, const GDNModel *m) {
    const size_t H = kH, I = kI, V = (size_t)e->vocab, L = (size_t)e->layers;
    const size_t per_layer = 4 * H * H + H * H + 2 * I * H + H * I;
    GDN_HIP(hipMalloc(&e->wmem, (L * per_layer + V * H) * 2));
    char *p = static_cast<char *>(e->wmem);
    std::vector<uint16_t> rows, part;
    for (size_t l = 0; l < L; ++l) {
        const GDNLayerWeights &w = m->layers[l];
        rows.resize(4 * H * H);
        const float *src[4] = {w.q_proj, w.k_proj, w.v_proj, w.g_proj};
        for (int s = 0; s < 4; ++s) {
            to_bf16(src[s], H * H, part);
            std::memcpy(rows.data() + s * H * H, part.data(), H * H * 2);
        }
        if (upload_tiled(rows, 4 * H, H, 2, p, e->w_qkvg[l])) return -1;
        to_bf16(w.o_proj, H * H, rows);
        if (upload_tiled(rows, H, H, kRtO, p, e->w_o[l])) return -1;
        std::vector<uint16_t> g16, u16;
        to_bf16(w.mlp_gate_proj, I * H, g16);
        to_bf16(w.mlp_up_proj, I * H, u16);
        rows.resize(2 * I * H);
        tile_gu(g16.data(), u16.data(), rows.data());
        GDN_HIP(hipMemcpy(p, rows.data(), rows.size() * 2, hipMemcpyHostToDevice));
        e->w_gu[l] = reinterpret_cast<const u32x4 *>(p);
        p += rows.size() * 2;
        to_bf16(w.mlp_down_proj, H * I, rows);
        if (upload_tiled(rows, H, I, kRtDown, p, e->w_down[l])) return -1;
    }
    to_bf16(m->lm_head, V * H, rows);
    if (upload_tiled(rows, V, H, lm_rt(e), p, e->w_lm)) return -1;
    // embeddings keep their top 16 bits (the batch-1 engine's import)
    std::vector<uint16_t> emb(V * H);
    for (size_t i = 0; i < V * H; ++i) {
        uint32_t b;
        std::memcpy(&b, m->embeddings + i, 4);
        emb[i] = (uint16_t)(b >> 16);
    }
    GDN_HIP(hipMalloc(&e->emb, emb.size() * 2));
    GDN_HIP(hipMemcpy(e->emb, emb.data(), emb.size() * 2, hipMemcpyHostToDevice));

    std::vector<float> aux(L * kAuxLayer + H, 0.0f);
    for (size_t l = 0; l < L; ++l) {
        const GDNLayerWeights &w = m->layers[l];
        float *a = aux.data() + l * kAuxLayer;
        std::memcpy(a + kAuxAttnNorm, w.attn_norm, H * 4);
        std::memcpy(a + kAuxMlpNorm, w.mlp_norm, H * 4);
        std::memcpy(a + kAuxONorm, w.o_norm, kHD * 4);
        std::memcpy(a + kAuxALog, w.a_log, kNH * 4);
        std::memcpy(a + kAuxDtBias, w.dt_bias, kNH * 4);
        std::memcpy(a + kAuxAB, w.a_proj, kNH * H * 4);
        std::memcpy(a + kAuxAB + kNH * H, w.b_proj, kNH * H * 4);
        std::memcpy(a + kAuxConv, w.q_conv, H * 4 * 4);
        std::memcpy(a + kAuxConv + H * 4, w.k_conv, H * 4 * 4);
        std::memcpy(a + kAuxConv + 2 * H * 4, w.v_conv, H * 4 * 4);
    }
    std::memcpy(aux.data() + L * kAuxLayer, m->final_norm, H * 4);
    GDN_HIP(hipMalloc(&e->aux, aux.size() * 4));
    GDN_HIP(hipMemcpy(e->aux, aux.data(), aux.size() * 4, hipMemcpyHostToDevice));
    return 0;
}

int b_alloc(GDNBatchEngine *e) {
    const size_t L = (size_t)e->layers, B = (size_t)e->streams, V = (size_t)e->vocab;
    GDN_HIP(hipMalloc(&e->state, L * B * kLayerState * 4));
    GDN_HIP(hipMemset(e->state, 0, L * B * kLayerState * 4));
    GDN_HIP(hipMalloc(&e->tails, L * B * kStreamTails * 2));
    GDN_HIP(hipMemset(e->tails, 0, L * B * kStreamTails * 2));
    const size_t G = (size_t)lm_wgs(e);
    const size_t act = kMaxB * (2 * kH + 3 * kH + kH + kH + 16 + kH + kSplitDown * kH + kH + V) + G * kMaxB;
    GDN_HIP(hipMalloc(&e->act, act * 4));
    GDN_HIP(hipMemset(e->act, 0, act * 4));
    float *p = e->act;
    e->h = p; p += 2 * kMaxB * kH;  // residual ping-pong (layer parity)
    e->qkv = p; p += kMaxB * 3 * kH;
    e->gate = p; p += kMaxB * kH;
    e->sgate = p; p += kMaxB * kH;
    e->bd = p; p += kMaxB * 16;
    e->attn = p; p += kMaxB * kH;
    e->ypart = p; p += (size_t)kSplitDown * kMaxB * kH;
    e->xn = p; p += kMaxB * kH;
    e->logits = p; p += kMaxB * V;
    e->part_val = p; p += G * kMaxB;
    GDN_HIP(hipMalloc(&e->part_idx, G * kMaxB * sizeof(int)));
    // X tiles: streams beyond n_streams stay zero
    GDN_HIP(hipMalloc(&e->x_h, (size_t)kMaxB * kH * 2));
    GDN_HIP(hipMalloc(&e->x_o, (size_t)kMaxB * kH * 2));
    GDN_HIP(hipMalloc(&e->x_d, (size_t)kMaxB * kI * 2));
    GDN_HIP(hipMemset(e->x_h, 0, (size_t)kMaxB * kH * 2));
    GDN_HIP(hipMemset(e->x_o, 0, (size_t)kMaxB * kH * 2));
    GDN_HIP(hipMemset(e->x_d, 0, (size_t)kMaxB * kI * 2));
    GDN_HIP(hipMalloc(&e->p_logits, (size_t)kMaxB * V * 4));
    GDN_HIP(hipMalloc(&e->p_tok, (size_t)kMaxB * sizeof(int)));
    // a step reads its tokens from and writes its argmaxes to host memory
    // directly
    GDN_HIP(hipHostMalloc(&e->tok_host, 2 * kMaxB * sizeof(int), hipHostMallocMapped | hipHostMallocCoherent));
    std::memset(e->tok_host, 0, 2 * kMaxB * sizeof(int));
    GDN_HIP(hipHostGetDevicePointer(reinterpret_cast<void **>(&e->tok_map), e->tok_host, 0));
    GDN_HIP(hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking));
    GDN_HIP(hipEventCreate(&e->ev0));
    GDN_HIP(hipEventCreate(&e->ev1));
    GDN_HIP(hipDeviceSynchronize());
    return 0;
}

// The residual entering layer l's attention block lives in buffer l & 1: the
// MLP norm updates it in place and the split a/b norm after the down
// projection writes the next layer's buffer.
float *b_resid(GDNBatchEngine *e, int l) { return e->h + (size_t)(l & 1) * kMaxB * kH; }

BNorm bnorm(GDNBatchEngine *e, const float *y, const float *w, uint16_t *x_out, int ab_layer, int l_in,
            int l_out) {
    BNorm p{};
    p.h_in = b_resid(e, l_in);
    p.h_out = b_resid(e, l_out);
    p.y = y;
    p.w = w;
    p.x_out = x_out;
    p.eps = e->eps;
    if (ab_layer >= 0) {
        float *a = b_aux(e, ab_layer);
        p.ab_w = a + kAuxAB;
        p.a_log = a + kAuxALog;
        p.dt_bias = a + kAuxDtBias;
        p.bd = e->bd;
    }
    return p;
}

// Kernel kinds of gdn_batch_profile_kernels, in output order.
enum { KB_EMBED, KB_QKVG, KB_RECUR, KB_ONORM, KB_O, KB_NORM, KB_GU, KB_DOWN, KB_LM, KB_ARGMAX, KB_KINDS };

void launch_embed(GDNBatchEngine *e, hipStream_t s) {
    BNorm p = bnorm(e, nullptr, b_aux(e, 0) + kAuxAttnNorm, e->x_h, 0, 0, 0);
    p.emb = e->emb;
    p.tok = e->tok_map;
    hipLaunchKernelGGL((k_bnorm<0, true, true>), dim3(e->streams, kAbSplit), dim3(kT), 0, s, p);
}
void launch_qkvg(GDNBatchEngine *e, int l, hipStream_t s) {
    BEpi ep{};
    ep.n_streams = e->streams;
    ep.n_rows = 4 * kH;
    ep.qkv = e->qkv;
    ep.gate = e->gate;
    ep.sgate = e->sgate;
    ep.tails = b_tails(e, l);
    ep.conv_w = b_aux(e, l) + kAuxConv;
    hipLaunchKernelGGL((k_bgemm<2, kKtH, 8, 1, EPI_QKVG>), dim3(4 * kH / 32), dim3(8 * 64), 0, s, e->w_qkvg[l],
                       reinterpret_cast<const u32x4 *>(e->x_h), ep);
}
void launch_recur(GDNBatchEngine *e, int l, hipStream_t s) {
    hipLaunchKernelGGL((k_brecur<kRecCols>), dim3(kNH * (kHD / kRecCols), e->streams), dim3(2 * kRecCols), 0, s,
                       e->qkv, e->bd, b_state(e, l), e->attn);
}
void launch_onorm(GDNBatchEngine *e, int l, hipStream_t s) {
    hipLaunchKernelGGL(k_bonorm<1>, dim3(kNH, e->streams), dim3(kT), 0, s, e->attn, e->gate, e->sgate,
                       b_aux(e, l) + kAuxONorm, e->eps, e->x_o, e->streams);
}
void launch_o(GDNBatchEngine *e, int l, hipStream_t s) {
    BEpi ep{};
    ep.n_streams = e->streams;
    ep.n_rows = kH;
    ep.y = e->ypart;
    hipLaunchKernelGGL((k_bgemm<kRtO, kKtH, 4, kSplitO, EPI_RAW>), dim3(kH / (16 * kRtO), kSplitO), dim3(kT), 0, s,
                       e->w_o[l], reinterpret_cast<const u32x4 *>(e->x_o), ep);
}
void launch_mlp_norm(GDNBatchEngine *e, int l, hipStream_t s) {
    const BNorm p = bnorm(e, e->ypart, b_aux(e, l) + kAuxMlpNorm, e->x_h, -1, l, l);
    hipLaunchKernelGGL((k_bnorm<kSplitO, false, false>), dim3(e->streams), dim3(kT), 0, s, p);
}
void launch_gu(GDNBatchEngine *e, int l, hipStream_t s) {
    hipLaunchKernelGGL(k_bgu<kGuWaves>, dim3(kGuWgs), dim3(kGuWaves * 64), 0, s, e->w_gu[l],
                       reinterpret_cast<const u32x4 *>(e->x_h), e->x_d, e->streams);
}
void launch_down(GDNBatchEngine *e, int l, hipStream_t s) {
    BEpi ep{};
    ep.n_streams = e->streams;
    ep.n_rows = kH;
    ep.y = e->ypart;
    hipLaunchKernelGGL((k_bgemm<kRtDown, kKtI, 4, kSplitDown, EPI_RAW>), dim3(kH / (16 * kRtDown), kSplitDown),
                       dim3(kT), 0, s, e->w_down[l], reinterpret_cast<const u32x4 *>(e->x_d), ep);
}
// After layer l's down projection: h = R(h + y), then the next layer's
// attention norm with its a/b rows, or the final norm.
void launch_layer_norm(GDNBatchEngine *e, int l, hipStream_t s) {
    if (l + 1 < e->layers) {
        const BNorm p = bnorm(e, e->ypart, b_aux(e, l + 1) + kAuxAttnNorm, e->x_h, l + 1, l, l + 1);
        hipLaunchKernelGGL((k_bnorm<kSplitDown, false, true>), dim3(e->streams, kAbSplit), dim3(kT), 0, s, p);
    } else {
        BNorm p = bnorm(e, e->ypart, e->aux + (size_t)e->layers * kAuxLayer, e->x_h, -1, l, l);
        p.xn_out = e->xn;
        hipLaunchKernelGGL((k_bnorm<kSplitDown, false, false>), dim3(e->streams), dim3(kT), 0, s, p);
    }
}
void launch_lm(GDNBatchEngine *e, hipStream_t s) {
    BEpi ep{};
    ep.n_streams = e->streams;
    ep.n_rows = e->vocab;
    ep.logits = e->logits;
    ep.part_val = e->part_val;
    ep.part_idx = e->part_idx;
    launch_lm_gemm(e, ep, e->x_h, s);
}
void launch_argmax(GDNBatchEngine *e, hipStream_t s) {
    hipLaunchKernelGGL(k_bargmax, dim3(e->streams), dim3(kT), 0, s, e->part_val, e->part_idx, lm_wgs(e),
                       e->tok_map + kMaxB);
}

void b_enqueue_step(GDNBatchEngine *e, hipStream_t s) {
    launch_embed(e, s);
    for (int l = 0; l < e->layers; ++l) {
        launch_qkvg(e, l, s);
        launch_recur(e, l, s);
        launch_onorm(e, l, s);
        launch_o(e, l, s);
        launch_mlp_norm(e, l, s);
        launch_gu(e, l, s);
        launch_down(e, l, s);
        launch_layer_norm(e, l, s);
    }
    launch_lm(e, s);
    launch_argmax(e, s);
}

int b_ensure_graph(GDNBatchEngine *e) {
    if (e->exec) return 0;
    GDN_HIP(hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal));
    b_enqueue_step(e, e->stream);
    GDN_HIP(hipStreamEndCapture(e->stream, &e->graph));
    GDN_HIP(hipGraphInstantiate(&e->exec, e->graph, nullptr, nullptr, 0));
    return 0;
}

// tokens[n_streams] in (host) -> step -> next tokens out (host).
int b_run_step(GDNBatchEngine *e, const int32_t *tokens, int32_t *next, float *inner_ms) {
    for (int i = 0; i < e->streams; ++i) {
        if (tokens[i] < 0 || tokens[i] >= e->vocab) {
            gdn_error("token id out of range");
            return -1;
        }
    }
    if (e->use_graph && b_ensure_graph(e) != 0) return -1;
    std::memcpy(e->tok_host, tokens, (size_t)e->streams * sizeof(int));  // read through tok_map
    if (inner_ms) GDN_HIP(hipEventRecord(e->ev0, e->stream));
    if (e->use_graph) {
        GDN_HIP(hipGraphLaunch(e->exec, e->stream));
    } else {
        b_enqueue_step(e, e->stream);
        GDN_HIP(hipGetLastError());
    }
    if (inner_ms) GDN_HIP(hipEventRecord(e->ev1, e->stream));
    GDN_HIP(hipStreamSynchronize(e->stream));  // k_bargmax wrote tok_host[kMaxB..]
    if (next) std::memcpy(next, e->tok_host + kMaxB, (size_t)e->streams * sizeof(int));
    if (inner_ms) GDN_HIP(hipEventElapsedTime(inner_ms, e->ev0, e->ev1));
    return 0;
}

// Prefill segment buffers for e->seg_tokens tokens (kept while the segment
// length stays).
int seg_alloc(GDNBatchEngine *e) {
    if (e->seg_cap == e->seg_tokens && e->seg_mem) return 0;
    GDN_HIP(hipStreamSynchronize(e->stream));
    (void)hipFree(e->seg_mem);
    e->seg_mem = nullptr;
    e->seg_cap = 0;
    const size_t T = (size_t)e->seg_tokens, chunks = T / kMaxB;
    const size_t floats = T * (2 * kH + 4 * kH + 3 * kH + kH + kH + 16 + kH + kH + kH + kNH + kH) +
                          2 * chunks * kNH * kMaxB * kMaxB;
    const size_t halves = T * (kH + kH + kI);
    const size_t bytes = floats * 4 + halves * 2 + T * sizeof(int);
    GDN_HIP(hipMalloc(&e->seg_mem, bytes));
    // X tiles of padded tokens are read by the GEMMs (their sums unused):
    // start them at zero, on the engine's stream (a plain hipMemset may
    // return before it completes, and the non-blocking stream would not
    // wait for it)
    GDN_HIP(hipMemsetAsync(e->seg_mem, 0, bytes, e->stream));
    float *p = static_cast<float *>(e->seg_mem);
    e->s_h = p; p += 2 * T * kH;
    e->s_y = p; p += 4 * T * kH;
    e->s_qkv = p; p += 3 * T * kH;
    e->s_gate = p; p += T * kH;
    e->s_sgate = p; p += T * kH;
    e->s_bd = p; p += T * 16;
    e->s_attn = p; p += T * kH;
    e->s_qn = p; p += T * kH;
    e->s_kn = p; p += T * kH;
    e->s_alpha = p; p += T * kNH;
    e->s_xn = p; p += T * kH;
    e->s_wyl = p; p += chunks * kNH * kMaxB * kMaxB;
    e->s_wym = p; p += chunks * kNH * kMaxB * kMaxB;
    uint16_t *q = reinterpret_cast<uint16_t *>(p);
    e->s_xh = q; q += T * kH;
    e->s_xo = q; q += T * kH;
    e->s_xd = q; q += T * kI;
    e->s_tok = reinterpret_cast<int *>(q);
    e->seg_cap = e->seg_tokens;
    return 0;
}

// A segment's norm: the residual of layer l's attention block in buffer
// l & 1 (as in the step), segment-sized.
BNorm seg_norm(GDNBatchEngine *e, const float *y, const float *w, uint16_t *x_out, int ab_layer, int l_in,
               int l_out) {
    BNorm p{};
    p.h_in = e->s_h + (size_t)(l_in & 1) * e->seg_cap * kH;
    p.h_out = e->s_h + (size_t)(l_out & 1) * e->seg_cap * kH;
    p.y = y;
    p.w = w;
    p.x_out = x_out;
    p.eps = e->eps;
    if (ab_layer >= 0) {
        float *a = b_aux(e, ab_layer);
        p.ab_w = a + kAuxAB;
        p.a_log = a + kAuxALog;
        p.dt_bias = a + kAuxDtBias;
        p.bd = e->s_bd;
    }
    return p;
}

// One prefill segment of n tokens (already in s_tok[0..n)) through stream
// `slot`'s state, layer by layer: the step's kernels with the tokens as the
// streams (k_pgemm / k_pgu in place of the step's GEMMs, k_bnorm + k_pab in
// place of the split a/b norm; same sums), the conv across the segment
// (k_pconv), and the recurrence chunk by chunk of 64 tokens, in token order
// (k_pqk, k_pscan) or in the WY form (k_wy_gram and k_wy_inv over every
// chunk at once, then k_wy_seq over the chunks in order).
// k_pgemm_a (the faster kernel once its grid fills the CUs) or k_pgemm (twice
// the workgroups at the same size, so the better one on short segments):
// the same sums either way.
bool pa_fills(int rows, int tiles) { return rows % kPaRows == 0 && (rows / kPaRows) * tiles >= 256; }

void enqueue_prefill_segment(GDNBatchEngine *e, int slot, int n, bool last, hipStream_t s) {
    const int blocks = (n + kMaxB - 1) / kMaxB, tiles = (n + kPgTok - 1) / kPgTok;
    const int pab_blocks = (n + kPabTok - 1) / kPabTok;
    // a norm's a/b rows and beta/decay, from its normalised copy in s_xn
    auto launch_ab = [&](int l_ab) {
        const float *a = b_aux(e, l_ab);
        hipLaunchKernelGGL(k_pab, dim3(kAbSplit, pab_blocks), dim3(kT), 0, s, e->s_xn, n, a + kAuxAB, a + kAuxALog,
                           a + kAuxDtBias, e->s_bd);
    };
    BNorm p0 = seg_norm(e, nullptr, b_aux(e, 0) + kAuxAttnNorm, e->s_xh, -1, 0, 0);
    p0.emb = e->emb;
    p0.tok = e->s_tok;
    p0.xn_out = e->s_xn;
    hipLaunchKernelGGL((k_bnorm<0, true, false>), dim3(n), dim3(kT), 0, s, p0);
    launch_ab(0);
    const u32x4 *xh = reinterpret_cast<const u32x4 *>(e->s_xh), *xo = reinterpret_cast<const u32x4 *>(e->s_xo),
                *xd = reinterpret_cast<const u32x4 *>(e->s_xd);
    for (int l = 0; l < e->layers; ++l) {
        float *st = b_state(e, l) + (size_t)slot * kLayerState;
        uint16_t *tl = b_tails(e, l) + (size_t)slot * kStreamTails;
        if (pa_fills(4 * kH, tiles))
            hipLaunchKernelGGL((k_pgemm_a<kKtH, 8, 1>), dim3(4 * kH / kPaRows, tiles), dim3(kPgW * 64), 0, s,
                               e->w_qkvg[l], xh, e->s_y, 4 * kH);
        else
            hipLaunchKernelGGL((k_pgemm<kKtH, 8, 1>), dim3(4 * kH / 128, tiles), dim3(kPgW * 64), 0, s,
                               e->w_qkvg[l], xh, e->s_y, 4 * kH);
        hipLaunchKernelGGL(k_pconv, dim3(4 * kH / 64, blocks), dim3(kConvT), 0, s, e->s_y, n, tl,
                           b_aux(e, l) + kAuxConv, e->s_qkv, e->s_gate, e->s_sgate);
        hipLaunchKernelGGL(k_pqk, dim3(kNH, (n + kQkTok - 1) / kQkTok), dim3(kT), 0, s, e->s_qkv, n, e->s_qn,
                           e->s_kn, e->s_alpha);
        if (e->prefill_mode == GDN_PREFILL_CHUNKED)
            hipLaunchKernelGGL(k_wy_gram, dim3(kNH, kMaxB / 16, blocks), dim3(kT), 0, s, e->s_qn, e->s_kn, e->s_bd,
                               n, e->s_wyl, e->s_wym);
        if (e->prefill_mode == GDN_PREFILL_CHUNKED)
            hipLaunchKernelGGL(k_wy_inv, dim3(kNH, blocks), dim3(64), 0, s, e->s_wyl);
        if (e->prefill_mode == GDN_PREFILL_CHUNKED)
            hipLaunchKernelGGL(k_wy_seq, dim3(kHD / kWyCols, kNH), dim3(kT), 0, s, e->s_qkv, e->s_qn, e->s_kn,
                               e->s_bd, e->s_wyl, e->s_wym, n, st, e->s_attn);
        else
            hipLaunchKernelGGL(k_pscan, dim3(kHD / kScanWgCols, kNH), dim3(kT), 0, s, e->s_qkv, e->s_qn, e->s_kn,
                               e->s_alpha, e->s_bd, n, st, e->s_attn);
        hipLaunchKernelGGL(k_bonorm<kOnTok>, dim3(kNH, (n + kOnTok - 1) / kOnTok), dim3(kT), 0, s, e->s_attn,
                           e->s_gate, e->s_sgate, b_aux(e, l) + kAuxONorm, e->eps, e->s_xo, n);
        hipLaunchKernelGGL((k_pgemm<kKtH, 4, kSplitO>), dim3(kH / 128, tiles), dim3(kPgW * 64), 0, s, e->w_o[l], xo,
                           e->s_y, kH);
        const BNorm pm = seg_norm(e, e->s_y, b_aux(e, l) + kAuxMlpNorm, e->s_xh, -1, l, l);
        hipLaunchKernelGGL((k_bnorm<1, false, false>), dim3(n), dim3(kT), 0, s, pm);
        hipLaunchKernelGGL(k_pgu, dim3(kGuWgs / 2, tiles), dim3(kPgW * 64), 0, s, e->w_gu[l], xh, e->s_xd, n);
        if (pa_fills(kH, tiles))
            hipLaunchKernelGGL((k_pgemm_a<kKtI, 4, kSplitDown>), dim3(kH / kPaRows, tiles), dim3(kPgW * 64), 0, s,
                               e->w_down[l], xd, e->s_y, kH);
        else
            hipLaunchKernelGGL((k_pgemm<kKtI, 4, kSplitDown>), dim3(kH / 128, tiles), dim3(kPgW * 64), 0, s,
                               e->w_down[l], xd, e->s_y, kH);
        if (l + 1 < e->layers) {
            BNorm pa = seg_norm(e, e->s_y, b_aux(e, l + 1) + kAuxAttnNorm, e->s_xh, -1, l, l + 1);
            pa.xn_out = e->s_xn;
            hipLaunchKernelGGL((k_bnorm<1, false, false>), dim3(n), dim3(kT), 0, s, pa);
            launch_ab(l + 1);
        } else {
            BNorm pf = seg_norm(e, e->s_y, e->aux + (size_t)e->layers * kAuxLayer, e->s_xh, -1, l, l);
            pf.xn_out = e->s_xn;
            hipLaunchKernelGGL((k_bnorm<1, false, false>), dim3(n), dim3(kT), 0, s, pf);
        }
    }
    if (!last) return;
    // the LM head over the last token block
    const int lb = blocks - 1, nl = n - lb * kMaxB;
    BEpi lm{};
    lm.n_streams = nl;
    lm.n_rows = e->vocab;
    lm.logits = e->p_logits;
    lm.part_val = e->part_val;
    lm.part_idx = e->part_idx;
    launch_lm_gemm(e, lm, e->s_xh + (size_t)lb * kMaxB * kH, s);
    hipLaunchKernelGGL(k_bargmax, dim3(nl), dim3(kT), 0, s, e->part_val, e->part_idx, lm_wgs(e), e->p_tok);
}

int b_prefill(GDNBatchEngine *e, int slot, const int32_t *prompt, uint32_t n_tokens, int32_t *seed) {
    for (uint32_t i = 0; i < n_tokens; ++i) {
        if (prompt[i] < 0 || prompt[i] >= e->vocab) {
            gdn_error("token id out of range");
            return -1;
        }
    }
    if (seg_alloc(e)) return -1;
    const uint32_t seg = (uint32_t)e->seg_cap;
    int n = 0;
    for (uint32_t off = 0; off < n_tokens; off += seg) {
        n = (int)std::min<uint32_t>(seg, n_tokens - off);
        GDN_HIP(hipMemcpyAsync(e->s_tok, prompt + off, (size_t)n * sizeof(int), hipMemcpyHostToDevice, e->stream));
        enqueue_prefill_segment(e, slot, n, off + (uint32_t)n == n_tokens, e->stream);
        GDN_HIP(hipGetLastError());
    }
    // the last position's logits, final hidden vector and token into the
    // stream's rows of the step buffers
    const int nl = n - ((n - 1) / kMaxB) * kMaxB;
    GDN_HIP(hipMemcpyAsync(e->logits + (size_t)slot * e->vocab, e->p_logits + (size_t)(nl - 1) * e->vocab,
                           (size_t)e->vocab * 4, hipMemcpyDeviceToDevice, e->stream));
    GDN_HIP(hipMemcpyAsync(e->xn + (size_t)slot * kH, e->s_xn + (size_t)(n - 1) * kH, (size_t)kH * 4,
                           hipMemcpyDeviceToDevice, e->stream));
    GDN_HIP(hipMemcpyAsync(e->tok_host + kMaxB + slot, e->p_tok + (nl - 1), sizeof(int), hipMemcpyDeviceToHost,
                           e->stream));
    GDN_HIP(hipStreamSynchronize(e->stream));
    if (seed) *seed = e->tok_host[kMaxB + slot];
    return 0;
}

void b_destroy(GDNBatchEngine *e) {
    if (!e) return;
    if (e->exec) (void)hipGraphExecDestroy(e->exec);
    if (e->graph) (void)hipGraphDestroy(e->graph);
    if (e->ev0) (void)hipEventDestroy(e->ev0);
    if (e->ev1) (void)hipEventDestroy(e->ev1);
    if (e->stream) (void)hipStreamDestroy(e->stream);
    (void)hipFree(e->wmem);
    (void)hipFree(e->emb);
    (void)hipFree(e->aux);
    (void)hipFree(e->state);
    (void)hipFree(e->tails);
    (void)hipFree(e->act);
    (void)hipFree(e->part_idx);
    (void)hipFree(e->x_h);
    (void)hipFree(e->x_o);
    (void)hipFree(e->x_d);
    (void)hipFree(e->p_logits);
    (void)hipFree(e->p_tok);
    (void)hipFree(e->seg_mem);
    if (e->tok_host) (void)hipHostFree(e->tok_host);
    delete e;
}

GDNBatchEngine *engine_of(const GDNBatchState *s) {
    if (!s || !s->engine) gdn_error("gdn: multi-stream state not initialised");
    return s ? s->engine : nullptr;
}

// Copy between one stream's [layers][per] block and the strided device array.
int stream_copy(float *dev, size_t per, int streams, int layers, uint32_t stream, float *host, bool to_dev) {
    const size_t width = per * 4, dpitch = (size_t)streams * per * 4;
    float *d = dev + (size_t)stream * per;
    if (to_dev)
        GDN_HIP(hipMemcpy2D(d, dpitch, host, width, width, (size_t)layers, hipMemcpyHostToDevice));
    else
        GDN_HIP(hipMemcpy2D(host, width, d, dpitch, width, (size_t)layers, hipMemcpyDeviceToHost));
    return 0;
}

// The conv tails of one stream: FP32 words on the host (the .gdnstate
// section layout), BF16 bits on the device.  Loading requires BF16-exact
// values, as the reference's head buffer does.
int tails_copy(uint16_t *dev, int streams, int layers, uint32_t stream, float *host, bool to_dev) {
    const size_t n = (size_t)layers * kStreamTails;
    std::vector<uint16_t> bits(n);
    const size_t width = kStreamTails * 2, dpitch = (size_t)streams * kStreamTails * 2;
    uint16_t *d = dev + (size_t)stream * kStreamTails;
    if (to_dev) {
        const size_t bad = gdn_first_non_bf16(host, n);
        if (bad != n) {
            gdn_report_non_bf16("multi-stream conv tail", host, bad);
            return -1;
        }
        for (size_t i = 0; i < n; ++i) {
            uint32_t u;
            std::memcpy(&u, host + i, 4);
            bits[i] = (uint16_t)(u >> 16);
        }
        GDN_HIP(hipMemcpy2D(d, dpitch, bits.data(), width, width, (size_t)layers, hipMemcpyHostToDevice));
    } else {
        GDN_HIP(hipMemcpy2D(bits.data(), width, d, dpitch, width, (size_t)layers, hipMemcpyDeviceToHost));
        for (size_t i = 0; i < n; ++i) {
            const uint32_t u = (uint32_t)bits[i] << 16;
            std::memcpy(host + i, &u, 4);
        }
    }
    return 0;
}

}  // namespace

// ================================================================== C ABI

extern "C" {

int gdn_batch_init(GDNBatchState *state, const GDNModel *model, uint32_t n_streams) {
    std::memset(state, 0, sizeof(*state));
    if (n_streams == 0 || n_streams > (uint32_t)kMaxB) {
        gdn_error("gdn: n_streams must be 1..64");
        return -1;
    }
    if (b_check_shape(&model->config) != 0) return -1;
    if (gdn_validate_bf16_exact_weights(model->weight_data, &model->config) != 0) {
        gdn_error("gdn: the multi-stream engine needs a BF16-exact checkpoint");
        return -1;
    }
    GDNBatchEngine *e = new GDNBatchEngine();
    e->layers = (int)model->config.num_layers;
    e->vocab = (int)model->config.vocab_size;
    e->streams = (int)n_streams;
    e->eps = model->config.norm_eps;
    if (b_alloc(e) != 0 || b_upload(e, model) != 0) {
        b_destroy(e);
        return -1;
    }
    state->engine = e;
    state->n_streams = n_streams;
    return 0;
}

void gdn_batch_free(GDNBatchState *state) {
    b_destroy(state->engine);
    std::memset(state, 0, sizeof(*state));
}

int gdn_batch_set_graph_mode(GDNBatchState *state, int use_graph) {
    GDNBatchEngine *e = engine_of(state);
    if (!e) return -1;
    e->use_graph = use_graph != 0;
    return 0;
}

int gdn_batch_decode_step(GDNBatchState *state, const int32_t *tokens, int32_t *next_tokens) {
    GDNBatchEngine *e = engine_of(state);
    if (!e) return -1;
    if (tokens == nullptr || next_tokens == nullptr) {
        gdn_error("gdn_batch_decode_step: tokens and next_tokens are required");
        return -1;
    }
    return b_run_step(e, tokens, next_tokens, nullptr);
}

int gdn_batch_read_tokens(const GDNBatchState *state, int32_t *tokens) {
    GDNBatchEngine *e = engine_of(state);
    if (!e) return -1;
    GDN_HIP(hipStreamSynchronize(e->stream));
    std::memcpy(tokens, e->tok_host + kMaxB, (size_t)e->streams * sizeof(int));
    return 0;
}

int gdn_batch_read_logits(const GDNBatchState *state, uint32_t stream, float *logits, size_t count) {
    GDNBatchEngine *e = engine_of(state);
    if (!e || stream >= (uint32_t)e->streams || count > (size_t)e->vocab) return -1;
    GDN_HIP(hipMemcpy(logits, e->logits + (size_t)stream * e->vocab, count * 4, hipMemcpyDeviceToHost));
    return 0;
}

int gdn_batch_read_final_hidden(const GDNBatchState *state, uint32_t stream, float *hidden, size_t count) {
    GDNBatchEngine *e = engine_of(state);
    if (!e || stream >= (uint32_t)e->streams || count > (size_t)kH) return -1;
    GDN_HIP(hipMemcpy(hidden, e->xn + (size_t)stream * kH, count * 4, hipMemcpyDeviceToHost));
    return 0;
}

int gdn_batch_load_stream_state(GDNBatchState *state, uint32_t stream, const float *recurrent,
                                size_t recurrent_floats, const float *conv_tails, size_t conv_floats) {
    GDNBatchEngine *e = engine_of(state);
    if (!e || stream >= (uint32_t)e->streams) return -1;
    if (recurrent && recurrent_floats != (size_t)e->layers * kLayerState) return -1;
    if (conv_tails && conv_floats != (size_t)e->layers * kStreamTails) return -1;
    // the tails first: they are checked (BF16-exact) before anything is written
    if (conv_tails && tails_copy(e->tails, e->streams, e->layers, stream, const_cast<float *>(conv_tails), true))
        return -1;
    if (recurrent && stream_copy(e->state, kLayerState, e->streams, e->layers, stream,
                                 const_cast<float *>(recurrent), true))
        return -1;
    return 0;
}

int gdn_batch_save_stream_state(const GDNBatchState *state, uint32_t stream, float *recurrent,
                                size_t recurrent_floats, float *conv_tails, size_t conv_floats) {
    GDNBatchEngine *e = engine_of(state);
    if (!e || stream >= (uint32_t)e->streams) return -1;
    if (recurrent && recurrent_floats != (size_t)e->layers * kLayerState) return -1;
    if (conv_tails && conv_floats != (size_t)e->layers * kStreamTails) return -1;
    if (recurrent && stream_copy(e->state, kLayerState, e->streams, e->layers, stream, recurrent, false)) return -1;
    if (conv_tails && tails_copy(e->tails, e->streams, e->layers, stream, conv_tails, false)) return -1;
    return 0;
}

int gdn_batch_set_prefill_mode(GDNBatchState *state, int mode) {
    GDNBatchEngine *e = engine_of(state);
    if (!e || (mode != GDN_PREFILL_SCAN && mode != GDN_PREFILL_CHUNKED)) return -1;
    e->prefill_mode = mode;
    return 0;
}

int gdn_batch_set_prefill_segment(GDNBatchState *state, uint32_t tokens) {
    GDNBatchEngine *e = engine_of(state);
    if (!e) return -1;
    if (tokens < (uint32_t)kPgTok || tokens > (uint32_t)kSegMax || tokens % kPgTok != 0) {
        gdn_error("gdn: a prefill segment is a multiple of 128 tokens, 128..32768");
        return -1;
    }
    e->seg_tokens = (int)tokens;
    return 0;
}

int gdn_batch_prefill(GDNBatchState *state, uint32_t stream, const int32_t *prompt, uint32_t n_tokens,
                      int32_t *seed_token) {
    GDNBatchEngine *e = engine_of(state);
    if (!e || stream >= (uint32_t)e->streams || n_tokens == 0 || !prompt) return -1;
    return b_prefill(e, (int)stream, prompt, n_tokens, seed_token);
}

int gdn_batch_run_teacher_forced(GDNBatchState *state, const int32_t *tokens, uint32_t n_steps,
                                 int32_t *argmax_out, float *inner_ms, float *outer_ms) {
    GDNBatchEngine *e = engine_of(state);
    if (!e) return -1;
    if (tokens == nullptr && n_steps > 0) {
        gdn_error("gdn_batch_run_teacher_forced: no tokens");
        return -1;
    }
    const size_t B = (size_t)e->streams;
    std::vector<int32_t> next(B);
    for (uint32_t i = 0; i < n_steps; ++i) {
        const auto t0 = std::chrono::steady_clock::now();
        if (b_run_step(e, tokens + (size_t)i * B, next.data(), inner_ms ? inner_ms + i : nullptr) != 0) return -1;
        const auto t1 = std::chrono::steady_clock::now();
        if (outer_ms) outer_ms[i] = std::chrono::duration<float, std::milli>(t1 - t0).count();
        if (argmax_out) std::memcpy(argmax_out + (size_t)i * B, next.data(), B * sizeof(int32_t));
    }
    return 0;
}

int gdn_batch_profile_kernels(GDNBatchState *state, uint32_t rounds, float *avg_us, uint32_t n_kinds) {
    GDNBatchEngine *e = engine_of(state);
    if (!e) return -1;
    for (uint32_t id = 0; id < n_kinds && id < (uint32_t)KB_KINDS; ++id) {
        GDN_HIP(hipStreamSynchronize(e->stream));
        GDN_HIP(hipEventRecord(e->ev0, e->stream));
        uint32_t launches = 0;
        for (uint32_t r = 0; r < rounds; ++r) {
            const int per_layer = (id == KB_EMBED || id == KB_LM || id == KB_ARGMAX) ? 1 : e->layers;
            for (int l = 0; l < per_layer; ++l, ++launches) {
                switch (id) {
                case KB_EMBED: launch_embed(e, e->stream); break;
                case KB_QKVG: launch_qkvg(e, l, e->stream); break;
                case KB_RECUR: launch_recur(e, l, e->stream); break;
                case KB_ONORM: launch_onorm(e, l, e->stream); break;
                case KB_O: launch_o(e, l, e->stream); break;
                case KB_NORM: launch_layer_norm(e, l, e->stream); break;
                case KB_GU: launch_gu(e, l, e->stream); break;
                case KB_DOWN: launch_down(e, l, e->stream); break;
                case KB_LM: launch_lm(e, e->stream); break;
                default: launch_argmax(e, e->stream); break;
                }
            }
        }
        GDN_HIP(hipEventRecord(e->ev1, e->stream));
        GDN_HIP(hipEventSynchronize(e->ev1));
        GDN_HIP(hipGetLastError());
        float ms = 0.0f;
        GDN_HIP(hipEventElapsedTime(&ms, e->ev0, e->ev1));
        avg_us[id] = launches ? 1000.0f * ms / (float)launches : 0.0f;
    }
    return 0;
}

int gdn_test_batch_gemm(const float *W, const float *X, uint32_t N, uint32_t K, float *Y) {
    const bool k_hidden = K == (uint32_t)kH;
    const uint32_t rows = 16u * (uint32_t)(k_hidden ? kRtO : kRtDown);  // rows per workgroup
    if (!(k_hidden || K == (uint32_t)kI) || N == 0 || (N % rows) != 0) {
        gdn_error("gdn_test_batch_gemm: K must be 2048 or 5632 and N a multiple of the workgroup's rows");
        return -1;
    }
    // the production configurations: o_proj's for K = 2048, down's for 5632
    const int splits = k_hidden ? kSplitO : kSplitDown;
    std::vector<uint16_t> wb, wt((size_t)N * K), xb;
    to_bf16(W, (size_t)N * K, wb);
    gdn_tile_bf16(wb.data(), N, K, k_hidden ? kRtO : kRtDown, wt.data());
    // X [64][K] in B-operand tiles: the A tiling of 64 rows in 4 row tiles
    to_bf16(X, (size_t)kMaxB * K, xb);
    std::vector<uint16_t> xt((size_t)kMaxB * K);
    gdn_tile_bf16(xb.data(), kMaxB, K, 4, xt.data());
    void *dw = nullptr, *dx = nullptr;
    float *dy = nullptr;
    GDN_HIP(hipMalloc(&dw, wt.size() * 2));
    GDN_HIP(hipMalloc(&dx, xt.size() * 2));
    GDN_HIP(hipMalloc(&dy, (size_t)splits * kMaxB * N * 4));
    GDN_HIP(hipMemcpy(dw, wt.data(), wt.size() * 2, hipMemcpyHostToDevice));
    GDN_HIP(hipMemcpy(dx, xt.data(), xt.size() * 2, hipMemcpyHostToDevice));
    BEpi ep{};
    ep.n_streams = kMaxB;
    ep.n_rows = (int)N;
    ep.y = dy;
    if (k_hidden)
        hipLaunchKernelGGL((k_bgemm<kRtO, kKtH, 4, kSplitO, EPI_RAW>), dim3(N / rows, kSplitO), dim3(kT), 0, 0,
                           static_cast<const u32x4 *>(dw), static_cast<const u32x4 *>(dx), ep);
    else
        hipLaunchKernelGGL((k_bgemm<kRtDown, kKtI, 4, kSplitDown, EPI_RAW>), dim3(N / rows, kSplitDown), dim3(kT),
                           0, 0, static_cast<const u32x4 *>(dw), static_cast<const u32x4 *>(dx), ep);
    GDN_HIP(hipGetLastError());
    std::vector<float> parts((size_t)splits * kMaxB * N);
    GDN_HIP(hipMemcpy(parts.data(), dy, parts.size() * 4, hipMemcpyDeviceToHost));
    // split sums in split order, as the consumers add them
    for (size_t i = 0; i < (size_t)kMaxB * N; ++i) {
        float v = parts[i];
        for (int sp = 1; sp < splits; ++sp) v = v + parts[(size_t)sp * kMaxB * N + i];
        Y[i] = v;
    }
    (void)hipFree(dw);
    (void)hipFree(dx);
    (void)hipFree(dy);
    return 0;
}

int gdn_test_prefill_gemm(int kind, const float *W, const float *X, uint32_t N, uint32_t T, float *Y,
                          float *Y_step) {
    // kind 0: q/k/v/g configuration (K 2048, 8 classes); 1: o_proj (K 2048,
    // 4 classes, 4 splits); 2: down (K 5632, 4 classes, 4 splits); 3:
    // gate/up + SwiGLU (W = gate then up rows, N = 5632)
    if (kind < 0 || kind > 3 || T == 0 || T > (uint32_t)kSegMax || N == 0 ||
        (kind < 3 && (N % 128) != 0) || (kind == 3 && N != (uint32_t)kI)) {
        gdn_error("gdn_test_prefill_gemm: kind 0..3, N a multiple of 128 (5632 for gate/up), T 1..32768");
        return -1;
    }
    const uint32_t K = kind == 2 ? (uint32_t)kI : (uint32_t)kH;
    const uint32_t blocks = (T + kMaxB - 1) / kMaxB, tp = (T + kPgTok - 1) / kPgTok * kPgTok;
    const size_t wn = (kind == 3 ? 2 : 1) * (size_t)N * K;
    std::vector<uint16_t> wb, wt(wn), xb, xt((size_t)tp * K, 0);
    to_bf16(W, wn, wb);
    if (kind == 3) tile_gu(wb.data(), wb.data() + (size_t)N * K, wt.data());
    else gdn_tile_bf16(wb.data(), N, K, 2, wt.data());
    std::vector<float> xpad((size_t)blocks * kMaxB * K, 0.0f);
    std::memcpy(xpad.data(), X, (size_t)T * K * 4);
    to_bf16(xpad.data(), xpad.size(), xb);
    for (uint32_t b = 0; b < blocks; ++b)
        gdn_tile_bf16(xb.data() + (size_t)b * kMaxB * K, kMaxB, K, 4, xt.data() + (size_t)b * kMaxB * K);
    const size_t out_elems = kind == 3 ? (size_t)tp * kI : (size_t)kSplitDown * tp * N;
    void *dw = nullptr, *dx = nullptr, *dy = nullptr, *dr = nullptr;
    GDN_HIP(hipMalloc(&dw, wt.size() * 2));
    GDN_HIP(hipMalloc(&dx, xt.size() * 2));
    GDN_HIP(hipMalloc(&dy, out_elems * 4));
    GDN_HIP(hipMalloc(&dr, out_elems * 4));
    GDN_HIP(hipMemset(dy, 0, out_elems * 4));
    GDN_HIP(hipMemset(dr, 0, out_elems * 4));
    GDN_HIP(hipMemcpy(dw, wt.data(), wt.size() * 2, hipMemcpyHostToDevice));
    GDN_HIP(hipMemcpy(dx, xt.data(), xt.size() * 2, hipMemcpyHostToDevice));
    const u32x4 *w4 = static_cast<const u32x4 *>(dw), *x4 = static_cast<const u32x4 *>(dx);
    const dim3 pg(N / 128, tp / kPgTok);
    const dim3 pa(N / kPaRows, tp / kPgTok);
    if (kind == 0 && N % kPaRows == 0)
        hipLaunchKernelGGL((k_pgemm_a<kKtH, 8, 1>), pa, dim3(kPgW * 64), 0, 0, w4, x4, (float *)dy, (int)N);
    if (kind == 0 && N % kPaRows != 0)
        hipLaunchKernelGGL((k_pgemm<kKtH, 8, 1>), pg, dim3(kPgW * 64), 0, 0, w4, x4, (float *)dy, (int)N);
    if (kind == 1)
        hipLaunchKernelGGL((k_pgemm<kKtH, 4, kSplitO>), pg, dim3(kPgW * 64), 0, 0, w4, x4, (float *)dy, (int)N);
    if (kind == 2 && N % kPaRows == 0)
        hipLaunchKernelGGL((k_pgemm_a<kKtI, 4, kSplitDown>), pa, dim3(kPgW * 64), 0, 0, w4, x4, (float *)dy, (int)N);
    if (kind == 2 && N % kPaRows != 0)
        hipLaunchKernelGGL((k_pgemm<kKtI, 4, kSplitDown>), pg, dim3(kPgW * 64), 0, 0, w4, x4, (float *)dy, (int)N);
    if (kind == 3)
        hipLaunchKernelGGL(k_pgu, dim3(kGuWgs / 2, tp / kPgTok), dim3(kPgW * 64), 0, 0, w4, x4,
                           static_cast<uint16_t *>(dy), (int)T);
    // the step's kernels, one 64-token block at a time
    for (uint32_t b = 0; b < blocks; ++b) {
        const u32x4 *xb4 = x4 + (size_t)b * kMaxB * K / 8;
        BEpi ep{};
        ep.n_streams = kMaxB;
        ep.n_rows = (int)N;
        ep.y = static_cast<float *>(dr) + (size_t)b * kSplitDown * kMaxB * N;
        if (kind == 0)
            hipLaunchKernelGGL((k_bgemm<2, kKtH, 8, 1, EPI_RAW>), dim3(N / 32), dim3(8 * 64), 0, 0, w4, xb4, ep);
        if (kind == 1)
            hipLaunchKernelGGL((k_bgemm<kRtO, kKtH, 4, kSplitO, EPI_RAW>), dim3(N / 32, kSplitO), dim3(kT), 0, 0,
                               w4, xb4, ep);
        if (kind == 2)
            hipLaunchKernelGGL((k_bgemm<kRtDown, kKtI, 4, kSplitDown, EPI_RAW>), dim3(N / 32, kSplitDown),
                               dim3(kT), 0, 0, w4, xb4, ep);
        if (kind == 3)
            hipLaunchKernelGGL(k_bgu<kGuWaves>, dim3(kGuWgs), dim3(kGuWaves * 64), 0, 0, w4, xb4,
                               static_cast<uint16_t *>(dr) + (size_t)b * kMaxB * kI, kMaxB);
    }
    GDN_HIP(hipGetLastError());
    GDN_HIP(hipDeviceSynchronize());
    if (kind == 3) {
        // both outputs are X tiles of width kI: untile the first T tokens
        std::vector<uint16_t> a((size_t)tp * kI), r((size_t)tp * kI);
        GDN_HIP(hipMemcpy(a.data(), dy, a.size() * 2, hipMemcpyDeviceToHost));
        GDN_HIP(hipMemcpy(r.data(), dr, r.size() * 2, hipMemcpyDeviceToHost));
        for (uint32_t m = 0; m < T; ++m)
            for (uint32_t k = 0; k < (uint32_t)kI; ++k) {
                const uint32_t kt = k >> 5, kk = k & 31, mm = m & 63;
                const size_t idx = (size_t)(m >> 6) * 64 * kI +
                                   (size_t)((((kt * 4 + (mm >> 4)) * 64 + ((kk >> 3) << 4) + (mm & 15)) << 3) + (kk & 7));
                const uint32_t ya = (uint32_t)a[idx] << 16, yr = (uint32_t)r[idx] << 16;
                std::memcpy(Y + (size_t)m * kI + k, &ya, 4);
                std::memcpy(Y_step + (size_t)m * kI + k, &yr, 4);
            }
    } else {
        std::vector<float> a((size_t)tp * N), r(out_elems);
        GDN_HIP(hipMemcpy(a.data(), dy, a.size() * 4, hipMemcpyDeviceToHost));
        GDN_HIP(hipMemcpy(r.data(), dr, r.size() * 4, hipMemcpyDeviceToHost));
        const int splits = kind == 0 ? 1 : kSplitDown;
        for (uint32_t m = 0; m < T; ++m)
            for (uint32_t n = 0; n < N; ++n) {
                const size_t base = (size_t)(m / kMaxB) * kSplitDown * kMaxB * N + (size_t)(m % kMaxB) * N + n;
                float v = r[base];
                for (int sp = 1; sp < splits; ++sp) v = v + r[base + (size_t)sp * kMaxB * N];
                Y[(size_t)m * N + n] = a[(size_t)m * N + n];
                Y_step[(size_t)m * N + n] = v;
            }
    }
    (void)hipFree(dw);
    (void)hipFree(dx);
    (void)hipFree(dy);
    (void)hipFree(dr);
    return 0;
}

}  // extern "C"

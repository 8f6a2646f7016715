// gdn_engine.hip -- device half of libgdn_amd.so: the CDNA4 (gfx950) kernels
// of one batch-1 GatedDeltaNet decode step, the device layout of weights and
// state, the captured per-token hipGraph, and the run-state entry points of
// include/gdn_amd.h.
//
// One decode step (token id -> argmax token id), per layer l:
//   k_qkvg     bf16 GEMV [4H x H] (q,k,v,g) + per-channel causal conv/SiLU
//              with the conv-tail shift, plus one extra workgroup for the
//              tiny a/b projections          gdn_model.cpp:3785-3797, :1501-1536,
//                                            :1543-1667, :5043-5130
//   k_recur    per (head, 64-column block): q/k L2 norm, beta/decay, the
//              fused Sk / Sq read pass, delta, o, and the rank-1 state update;
//              the last block of a head applies the output RMSNorm * gate
//                                            :2376-2933, :3226-3349
//   k_gemv_res o_proj GEMV; the last block adds the residual and applies the
//              MLP RMSNorm                   :3803-3814, :3379-3450
//   k_gu       gate/up GEMV (rows interleaved 4+4) with the SwiGLU epilogue
//                                            :3815-3826, :4751-4767
//   k_gemv_res down GEMV; the last block adds the residual and applies the
//              next layer's attention RMSNorm (the final norm after the last)
//                                            :3827-3842
// then k_lm: LM-head GEMV writing FP32 logits and a two-stage argmax
// (:3857-3890, :4778-4931).  k_embed opens the step (:3716-3740, :1394-1474).
//
// Arithmetic follows the reference's all-BF16 contract bit for bit (products
// rounded to BF16 with DAZ/FTZ, tree16 + four-bank reduction, every operator
// output rounded to BF16); exp/log1p are evaluated through double precision
// (correctly rounded float results), the only place the reference's glibc
// calls can differ.
#include <hip/hip_runtime.h>

#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "gdn_amd.h"
#include "gdn_internal.h"

#define GDN_HIP(call)                                                              \
    do {                                                                           \
        hipError_t e_ = (call);                                                    \
        if (e_ != hipSuccess) {                                                    \
            std::fprintf(stderr, "gdn: %s failed: %s (%s:%d)\n", #call,            \
                         hipGetErrorString(e_), __FILE__, __LINE__);               \
            return -1;                                                             \
        }                                                                          \
    } while (0)

namespace gdn {

constexpr int kH = 2048;   // hidden
constexpr int kNH = 8;     // heads
constexpr int kHD = 256;   // head dim (dk = dv)
constexpr int kI = 5632;   // MLP intermediate
constexpr int kT = 256;    // threads per workgroup (4 wave64)
constexpr int kMaxLayers = 24;
constexpr int kTailStripe = 6144;  // floats reserved per (layer, q|k|v) conv-tail stripe

// Row blocking per GEMV (rows per workgroup).
constexpr int kRbQkvg = 8;
constexpr int kRbO = 4;
constexpr int kRbGu = 8;   // 4 gate rows + the 4 matching up rows
constexpr int kRbDown = 4;
constexpr int kRbLm = 8;
constexpr int kRbTest = 8;
constexpr int kCB = 64;    // state columns per recurrence workgroup

enum { kRef = GDN_CONTRACT_REF, kBf16w = GDN_CONTRACT_BF16W_FP32S, kFp32 = GDN_CONTRACT_FP32 };

// Per-layer block of small FP32 weights (norms, scalars, a/b rows, conv taps).
constexpr int kAuxAttnNorm = 0;
constexpr int kAuxMlpNorm = kH;
constexpr int kAuxONorm = 2 * kH;
constexpr int kAuxALog = 2 * kH + kHD;
constexpr int kAuxDtBias = kAuxALog + kNH;
constexpr int kAuxAB = kAuxALog + 16;
constexpr int kAuxConv = kAuxAB + 2 * kNH * kH;
constexpr int kAuxLayer = kAuxConv + 3 * kH * 4;

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Smallest nonzero |w| of a matrix (after DAZ) and whether any is not finite.
struct WInfo {
    float min_abs;
    int nonfinite;
};

// ---------------------------------------------------------------- scalar math

__device__ __forceinline__ uint32_t f2u(float f) { return __float_as_uint(f); }
__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }

// fp32_to_bf16_rne, gdn_model.cpp:309-320 (canonical NaN, infinities kept).
__device__ __forceinline__ float rne_bf16(float x) {
    const uint32_t b = f2u(x), mag = b & 0x7fffffffu;
    if (mag >= 0x7f800000u) {
        if (mag == 0x7f800000u) return x;
        return u2f((b & 0x80000000u) ? 0xffc00000u : 0x7fc00000u);
    }
    return u2f((b + 0x7fffu + ((b >> 16) & 1u)) & 0xffff0000u);
}

template <int C>
__device__ __forceinline__ float R(float x) {
    if constexpr (C == kFp32) return x;
    else return rne_bf16(x);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b16) { return u2f(b16 << 16); }

// exp and log1p through double: correctly rounded float results.
__device__ __forceinline__ float exp_cr(float x) { return (float)exp((double)x); }
__device__ __forceinline__ float log1p_cr(float x) { return (float)log1p((double)x); }

// gdn_sigmoid / gdn_silu / gdn_softplus, gdn_model.cpp:1307-1330.
__device__ __forceinline__ float sigmoid_ref(float x) {
    if (x >= 0.0f) {
        const float z = exp_cr(-x);
        return 1.0f / (1.0f + z);
    }
    const float z = exp_cr(x);
    return z / (1.0f + z);
}
__device__ __forceinline__ float silu_ref(float x) { return x * sigmoid_ref(x); }
__device__ __forceinline__ float softplus_ref(float x) {
    if (x > 20.0f) return x;
    if (x < -20.0f) return exp_cr(x);
    return log1p_cr(exp_cr(x));
}

// Balanced pairwise sum of 16 contiguous values (gemv32_tree16).
__device__ __forceinline__ float tree16(const float *p) {
    const float s0 = p[0] + p[1], s1 = p[2] + p[3], s2 = p[4] + p[5], s3 = p[6] + p[7];
    const float s4 = p[8] + p[9], s5 = p[10] + p[11], s6 = p[12] + p[13], s7 = p[14] + p[15];
    const float a0 = s0 + s1, a1 = s2 + s3, a2 = s4 + s5, a3 = s6 + s7;
    const float b0 = a0 + a1, b1 = a2 + a3;
    return b0 + b1;
}

// XOR butterfly over a wave64: every lane ends with the balanced pairwise
// sum of the 64 values (the lower six levels of gdn_tree_reduce_256).
__device__ __forceinline__ float wave_tree64(float v) {
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) v = v + __shfl_xor(v, m);
    return v;
}

// The native BF16 product with every special case of gdn_model.cpp:401-462:
// DAZ inputs, canonical NaN, signed infinities/zeros, FTZ below 0x007fc000.
__device__ __forceinline__ float native_exact(uint32_t w, float xf) {
    const uint32_t x = f2u(xf) >> 16;
    const uint32_t ew = (w >> 7) & 0xffu, fw = w & 0x7fu;
    const uint32_t ex = (x >> 7) & 0xffu, fx = x & 0x7fu;
    const bool w_nan = ew == 0xffu && fw, x_nan = ex == 0xffu && fx;
    const bool w_inf = ew == 0xffu && !fw, x_inf = ex == 0xffu && !fx;
    const bool w_zero = ew == 0, x_zero = ex == 0;
    const uint32_t sign = (w ^ x) & 0x8000u;
    if (w_nan || x_nan || (w_inf && x_zero) || (x_inf && w_zero)) return u2f(0x7fc00000u);
    if (w_inf || x_inf) return u2f((sign | 0x7f80u) << 16);
    if (w_zero || x_zero) return u2f(sign << 16);
    const float prod = bf16_bits_to_f32(w) * bf16_bits_to_f32(x);
    const uint32_t pb = f2u(prod), mag = pb & 0x7fffffffu;
    if (mag == 0x7f800000u) return prod;
    if (mag < 0x007fc000u) return u2f(pb & 0x80000000u);
    const uint32_t r = (pb + 0x7fffu + ((pb >> 16) & 1u)) & 0xffff0000u;
    if ((r & 0x7f800000u) == 0) return u2f(r & 0x80000000u);
    return u2f(r);
}

// Two native products when every operand is finite and normal and no
// product can fall below the flush threshold: the FP32 product is then
// exact, so one v_cvt_pk_bf16_f32 (round to nearest even) finishes both.
__device__ __forceinline__ void native_pair_fast(uint32_t w2, float x0, float x1, float &p0,
                                                 float &p1) {
    const float a = u2f(w2 << 16) * x0;
    const float b = u2f(w2 & 0xffff0000u) * x1;
    const bf16x2 r = __builtin_convertvector((f32x2){a, b}, bf16x2);
    const uint32_t rb = __builtin_bit_cast(uint32_t, r);
    p0 = u2f(rb << 16);
    p1 = u2f(rb & 0xffff0000u);
}

__device__ __forceinline__ void lds_load16(const float *src, float *v) {
    const f32x4 *s4 = reinterpret_cast<const f32x4 *>(src);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const f32x4 t = s4[q];
        v[4 * q + 0] = t.x;
        v[4 * q + 1] = t.y;
        v[4 * q + 2] = t.z;
        v[4 * q + 3] = t.w;
    }
}

__device__ __forceinline__ float coherent_load(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------------------ GEMV core
//
// A workgroup owns RB consecutive rows of the device matrix (stored
// row-major, so the block is one contiguous stream).  Work item f is one
// 16-column half-beat of one row: row f / (K/16), half-beat f % (K/16), at
// element offset 16 f of the block -- consecutive threads read consecutive
// 32-byte (BF16) or 64-byte (FP32) pieces.  Each item's 16 products are
// reduced in-lane with tree16 into LDS; then lanes 0..4RB-1 of wave 0 each
// run one of the reference's four bank chains (lower/upper half x even/odd
// beat, beat order, from +0.0f) and two XOR shuffles form
// (even_lo + even_hi) + (odd_lo + odd_hi).

template <int K>
struct Hb {
    static constexpr int HB = K / 16;     // half-beats per row
    static constexpr int HBP = HB + 4;    // padded LDS row stride
    static constexpr int NB = K / 32;     // 32-column beats per row
};

// Copy x into LDS and decide whether the fast product path is exact for
// this call: BF16 contracts only; all activations finite and normal (or
// zero), weights finite, and min|x| * min|w| >= 2^-125.
template <int C>
__device__ bool stage_x(const float *__restrict__ x, int K, float *xs, WInfo wi, float *red,
                        int *redi) {
    int bad = 0;
    float mn = INFINITY;
    for (int i = threadIdx.x; i < K; i += kT) {
        const float v = x[i];
        xs[i] = v;
        if constexpr (C != kFp32) {
            const uint32_t m = f2u(v) & 0x7fffffffu;
            if (m >= 0x7f800000u || (m != 0u && m < 0x00800000u)) bad = 1;
            else if (m != 0u) mn = fminf(mn, u2f(m));
        }
    }
    if constexpr (C == kFp32) {
        __syncthreads();
        return false;
    } else {
#pragma unroll
        for (int m = 1; m < 64; m <<= 1) mn = fminf(mn, __shfl_xor(mn, m));
        const int wbad = __any(bad) ? 1 : 0;
        const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
        if (lane == 0) {
            red[w] = mn;
            redi[w] = wbad;
        }
        __syncthreads();
        const float gm = fminf(fminf(red[0], red[1]), fminf(red[2], red[3]));
        const int gb = redi[0] | redi[1] | redi[2] | redi[3];
        if (gb || wi.nonfinite) return false;
        if (gm == INFINITY || wi.min_abs == INFINITY) return true;
        return (double)gm * (double)wi.min_abs >= 0x1p-125;
    }
}

template <int K, int RB, int C, bool FAST>
__device__ __forceinline__ void gemv_partials(const void *__restrict__ wblk, const float *xs,
                                              float *part) {
    constexpr int HB = Hb<K>::HB, HBP = Hb<K>::HBP;
    constexpr int ITEMS = RB * HB;
    constexpr int NIT = (ITEMS + kT - 1) / kT;
    constexpr bool kFull = (ITEMS % kT) == 0;
    const int t = threadIdx.x;
    const u32x4 *W = reinterpret_cast<const u32x4 *>(wblk);
    if constexpr (C != kFp32) {
        u32x4 wv[NIT][2];
#pragma unroll
        for (int i = 0; i < NIT; ++i) {
            const int f = t + kT * i;
            if (kFull || f < ITEMS) {
                wv[i][0] = __builtin_nontemporal_load(W + 2 * f);
                wv[i][1] = __builtin_nontemporal_load(W + 2 * f + 1);
            }
        }
#pragma unroll
        for (int i = 0; i < NIT; ++i) {
            const int f = t + kT * i;
            if (kFull || f < ITEMS) {
                const int row = f / HB, hb = f - row * HB;
                float xv[16], p[16];
                lds_load16(xs + hb * 16, xv);
                const uint32_t w8[8] = {wv[i][0].x, wv[i][0].y, wv[i][0].z, wv[i][0].w,
                                        wv[i][1].x, wv[i][1].y, wv[i][1].z, wv[i][1].w};
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    if constexpr (FAST) {
                        native_pair_fast(w8[e], xv[2 * e], xv[2 * e + 1], p[2 * e], p[2 * e + 1]);
                    } else {
                        p[2 * e] = native_exact(w8[e] & 0xffffu, xv[2 * e]);
                        p[2 * e + 1] = native_exact(w8[e] >> 16, xv[2 * e + 1]);
                    }
                }
                part[row * HBP + hb] = tree16(p);
            }
        }
    } else {
        constexpr int BATCH = 4;
#pragma unroll
        for (int i0 = 0; i0 < NIT; i0 += BATCH) {
            u32x4 wv[BATCH][4];
#pragma unroll
            for (int b = 0; b < BATCH; ++b) {
                const int i = i0 + b, f = t + kT * i;
                if (i < NIT && (kFull || f < ITEMS)) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) wv[b][q] = __builtin_nontemporal_load(W + 4 * f + q);
                }
            }
#pragma unroll
            for (int b = 0; b < BATCH; ++b) {
                const int i = i0 + b, f = t + kT * i;
                if (i < NIT && (kFull || f < ITEMS)) {
                    const int row = f / HB, hb = f - row * HB;
                    float xv[16], p[16];
                    lds_load16(xs + hb * 16, xv);
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        p[4 * q + 0] = u2f(wv[b][q].x) * xv[4 * q + 0];
                        p[4 * q + 1] = u2f(wv[b][q].y) * xv[4 * q + 1];
                        p[4 * q + 2] = u2f(wv[b][q].z) * xv[4 * q + 2];
                        p[4 * q + 3] = u2f(wv[b][q].w) * xv[4 * q + 3];
                    }
                    part[row * HBP + hb] = tree16(p);
                }
            }
        }
    }
}

// Wave 0 only.  Lane 4r ends with row r's result.
template <int K, int RB>
__device__ __forceinline__ float gemv_chain(const float *part) {
    constexpr int HBP = Hb<K>::HBP, NB = Hb<K>::NB;
    static_assert(RB * 4 <= 64, "one wave runs every bank chain");
    const int lane = threadIdx.x;
    float acc = 0.0f;
    if (lane < RB * 4) {
        const int row = lane >> 2, parity = (lane >> 1) & 1, half = lane & 1;
        const float *pr = part + row * HBP + half;
#pragma unroll 8
        for (int b = parity; b < NB; b += 2) acc = acc + pr[2 * b];
    }
    const float s = acc + __shfl_xor(acc, 1);
    return s + __shfl_xor(s, 2);
}

template <int K, int RB, int C>
__device__ __forceinline__ float gemv_block(const void *__restrict__ W, const float *__restrict__ x,
                                            WInfo wi, float *xs, float *part, float *red,
                                            int *redi) {
    const bool fast = stage_x<C>(x, K, xs, wi, red, redi);
    constexpr size_t esz = (C == kFp32) ? 4 : 2;
    const char *wblk = reinterpret_cast<const char *>(W) + (size_t)blockIdx.x * RB * K * esz;
    if (fast) gemv_partials<K, RB, C, true>(wblk, xs, part);
    else gemv_partials<K, RB, C, false>(wblk, xs, part);
    __syncthreads();
    float y = 0.0f;
    if (threadIdx.x < 64) y = gemv_chain<K, RB>(part);
    return y;
}

// Sum of squares of 2048 LDS values in the norm order (16-value chunks summed
// sequentially, chunk sums added sequentially), then
// out = R((x * scale) * w) with scale = 1/sqrtf(sum/2048 + eps)
// (gdn_rmsnorm_rows_bf16 / gdn_residual_rmsnorm_bf16).
template <int C>
__device__ void block_rmsnorm_h(const float *xl, const float *__restrict__ w, float *__restrict__ out,
                                float eps, float *scratch) {
    const int t = threadIdx.x;
    if (t < kH / 16) {
        float s = 0.0f;
#pragma unroll
        for (int kk = 0; kk < 16; ++kk) {
            const float v = xl[16 * t + kk];
            s += v * v;
        }
        scratch[t] = s;
    }
    __syncthreads();
    float sum = 0.0f;
    for (int i = 0; i < kH / 16; ++i) sum += scratch[i];
    const float scale = 1.0f / __builtin_sqrtf(sum / (float)kH + eps);
    for (int i = t; i < kH; i += kT) out[i] = R<C>(xl[i] * scale * w[i]);
}

// Arrival counter for "last workgroup finishes the step".  Call after the
// block's global results are stored.  Returns true in exactly one block.
__device__ __forceinline__ bool last_block_arrives(unsigned *cnt, unsigned total, int *flag) {
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned ticket = atomicAdd(cnt, 1u);
        *flag = (ticket == total - 1u) ? 1 : 0;
        if (*flag) *cnt = 0u;  // ready for the next launch
    }
    __syncthreads();
    if (*flag) __threadfence();
    return *flag != 0;
}

// -------------------------------------------------------------------- kernels

// Embedding row (or a given residual row) -> residual stream -> RMSNorm.
template <int C>
__global__ __launch_bounds__(kT) void k_embed(const int *__restrict__ tok_in, int vocab,
                                              const void *__restrict__ emb,
                                              const float *__restrict__ resid_in,
                                              float *__restrict__ ws_x, float *__restrict__ resid,
                                              const float *__restrict__ norm_w,
                                              float *__restrict__ xn, float eps) {
    __shared__ __attribute__((aligned(16))) float xl[kH];
    __shared__ float scratch[kH / 16];
    if (resid_in == nullptr) {
        int tok = tok_in[0];
        if (tok < 0 || tok >= vocab) tok = 0;  // the host rejects these first
        for (int i = threadIdx.x; i < kH; i += kT) {
            float e;
            if constexpr (C == kFp32) {
                e = reinterpret_cast<const float *>(emb)[(size_t)tok * kH + i];
            } else {
                e = bf16_bits_to_f32(reinterpret_cast<const uint16_t *>(emb)[(size_t)tok * kH + i]);
            }
            ws_x[i] = e;
            const float r = R<C>(e);
            resid[i] = r;
            xl[i] = r;
        }
    } else {
        for (int i = threadIdx.x; i < kH; i += kT) {
            const float r = resid_in[i];
            resid[i] = r;
            xl[i] = r;
        }
    }
    __syncthreads();
    block_rmsnorm_h<C>(xl, norm_w, xn, eps, scratch);
}

// The tiny a/b projections: 16 rows (a 0..7, b 8..15) of FP32 products,
// acc = (acc + tree16(lo)) + tree16(hi) per beat (gdn_gemv_tiny_ab).
template <int C>
__device__ void ab_block(const float *__restrict__ abw, const float *xs, float *part,
                         float *__restrict__ ab) {
    constexpr int HB = Hb<kH>::HB, HBP = Hb<kH>::HBP;
#pragma unroll
    for (int i = 0; i < (16 * HB) / kT; ++i) {
        const int f = threadIdx.x + kT * i;
        const int row = f / HB, hb = f - row * HB;
        const f32x4 *w4 = reinterpret_cast<const f32x4 *>(abw + (size_t)row * kH + hb * 16);
        float p[16];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const f32x4 wq = w4[q];
            p[4 * q + 0] = xs[hb * 16 + 4 * q + 0] * wq.x;
            p[4 * q + 1] = xs[hb * 16 + 4 * q + 1] * wq.y;
            p[4 * q + 2] = xs[hb * 16 + 4 * q + 2] * wq.z;
            p[4 * q + 3] = xs[hb * 16 + 4 * q + 3] * wq.w;
        }
        part[row * HBP + hb] = tree16(p);
    }
    __syncthreads();
    if (threadIdx.x < 16) {
        const float *pr = part + threadIdx.x * HBP;
        float acc = 0.0f;
        for (int j = 0; j < HB / 2; ++j) acc = (acc + pr[2 * j]) + pr[2 * j + 1];
        ab[threadIdx.x] = R<C>(acc);
    }
}

// q/k/v/g projection + conv/SiLU + conv-tail shift; last block: a/b.
template <int C, int RB>
__global__ __launch_bounds__(kT) void k_qkvg(const void *__restrict__ W, const float *__restrict__ x,
                                             WInfo wi, const float *__restrict__ aux,
                                             float *__restrict__ tails, float *__restrict__ qkv,
                                             float *__restrict__ gate, float *__restrict__ ab) {
    __shared__ __attribute__((aligned(16))) float xs[kH];
    __shared__ __attribute__((aligned(16))) float part[16 * Hb<kH>::HBP];
    __shared__ float red[4];
    __shared__ int redi[4];
    constexpr int nmain = 4 * kH / RB;
    if (blockIdx.x == nmain) {
        (void)stage_x<C>(x, kH, xs, wi, red, redi);
        ab_block<C>(aux + kAuxAB, xs, part, ab);
        return;
    }
    const float y = gemv_block<kH, RB, C>(W, x, wi, xs, part, red, redi);
    const int lane = threadIdx.x;
    if (lane < 64 && (lane & 3) == 0 && (lane >> 2) < RB) {
        const int r = blockIdx.x * RB + (lane >> 2);
        const float yv = R<C>(y);
        if (r < 3 * kH) {
            const int kind = r / kH, c = r - kind * kH;
            const float *cw = aux + kAuxConv + ((size_t)kind * kH + c) * 4;
            float t0, t1, t2;
            if constexpr (C == kFp32) {
                float *tl = tails + (size_t)kind * kTailStripe;
                t0 = tl[c];
                t1 = tl[kH + c];
                t2 = tl[2 * kH + c];
                tl[c] = t1;
                tl[kH + c] = t2;
                tl[2 * kH + c] = yv;
            } else {
                uint16_t *tl = reinterpret_cast<uint16_t *>(tails + (size_t)kind * kTailStripe);
                const uint16_t b0 = tl[c], b1 = tl[kH + c], b2 = tl[2 * kH + c];
                t0 = bf16_bits_to_f32(b0);
                t1 = bf16_bits_to_f32(b1);
                t2 = bf16_bits_to_f32(b2);
                tl[c] = b1;
                tl[kH + c] = b2;
                tl[2 * kH + c] = (uint16_t)(f2u(yv) >> 16);
            }
            const float s = t0 * cw[0] + t1 * cw[1] + t2 * cw[2] + yv * cw[3];
            qkv[r] = R<C>(silu_ref(s));
        } else {
            gate[r - 3 * kH] = yv;
        }
    }
}

// Gated delta rule for one head and CB state columns.
template <int C, int CB>
__global__ __launch_bounds__(kT) void k_recur(
    const float *__restrict__ qp, const float *__restrict__ kp, const float *__restrict__ vp,
    const float *__restrict__ a, const float *__restrict__ b, const float *__restrict__ a_log,
    const float *__restrict__ dt_bias, void *__restrict__ state, float *__restrict__ attn,
    const float *__restrict__ gate, const float *__restrict__ onorm_w, float *__restrict__ og,
    unsigned *__restrict__ cnt, float eps, int do_onorm) {
    static_assert(CB <= 64 && (CB % 8) == 0, "one wave owns the column chains");
    __shared__ float qn[kHD], kn[kHD];
    __shared__ __attribute__((aligned(16))) float tile[kHD * CB];
    __shared__ float dl[CB];
    __shared__ float red[8], red2[4], sc[2];
    __shared__ int flag;
    const int h = blockIdx.y, c0 = blockIdx.x * CB, t = threadIdx.x;
    const int lane = t & 63, w = t >> 6;

    // q/k L2 norms (gdn_tree_reduce_256 order: four wave butterflies, then
    // (w0 + w1) + (w2 + w3)).
    const float q = qp[h * kHD + t], k = kp[h * kHD + t];
    const float qs = wave_tree64(q * q), ks = wave_tree64(k * k);
    if (lane == 0) {
        red[w] = qs;
        red[4 + w] = ks;
    }
    __syncthreads();
    const float q_sq = (red[0] + red[1]) + (red[2] + red[3]);
    const float k_sq = (red[4] + red[5]) + (red[6] + red[7]);
    const float q_inv = 1.0f / __builtin_sqrtf(q_sq + 1e-6f);
    const float k_inv = 1.0f / __builtin_sqrtf(k_sq + 1e-6f);
    const float qv = q * q_inv, kv = k * k_inv;
    qn[t] = qv;
    kn[t] = kv;
    const float ap = wave_tree64(qv * kv);
    if (lane == 0) red2[w] = ap;
    if (t == 0) {
        sc[0] = sigmoid_ref(b[h]);
        const float decay_in = a[h] + dt_bias[h];
        const float decay_val = -exp_cr(a_log[h]) * softplus_ref(decay_in);
        sc[1] = exp_cr(decay_val);
    }

    // Stage the 256 x CB state tile.
    const size_t sbase = (size_t)h * kHD * kHD + c0;
    if constexpr (C == kRef) {
        constexpr int PER_ROW = CB / 8;  // 8 BF16 per 16-byte load
        const uint16_t *S = reinterpret_cast<const uint16_t *>(state);
#pragma unroll
        for (int i = 0; i < (kHD * PER_ROW) / kT; ++i) {
            const int u = t + kT * i, row = u / PER_ROW, c8 = u - row * PER_ROW;
            const u32x4 v = *reinterpret_cast<const u32x4 *>(S + sbase + (size_t)row * kHD + c8 * 8);
            f32x4 lo, hi;
            lo.x = u2f(v.x << 16); lo.y = u2f(v.x & 0xffff0000u);
            lo.z = u2f(v.y << 16); lo.w = u2f(v.y & 0xffff0000u);
            hi.x = u2f(v.z << 16); hi.y = u2f(v.z & 0xffff0000u);
            hi.z = u2f(v.w << 16); hi.w = u2f(v.w & 0xffff0000u);
            f32x4 *dst = reinterpret_cast<f32x4 *>(tile + row * CB + c8 * 8);
            dst[0] = lo;
            dst[1] = hi;
        }
    } else {
        constexpr int PER_ROW = CB / 4;
        const float *S = reinterpret_cast<const float *>(state);
#pragma unroll
        for (int i = 0; i < (kHD * PER_ROW) / kT; ++i) {
            const int u = t + kT * i, row = u / PER_ROW, c4 = u - row * PER_ROW;
            *reinterpret_cast<f32x4 *>(tile + row * CB + c4 * 4) =
                *reinterpret_cast<const f32x4 *>(S + sbase + (size_t)row * kHD + c4 * 4);
        }
    }
    __syncthreads();
    const float alpha = (red2[0] + red2[1]) + (red2[2] + red2[3]);
    const float beta = sc[0], decay = sc[1];

    // Read pass: column chains in row order (one lane per column).
    if (t < CB) {
        float r = 0.0f, p = 0.0f;
#pragma unroll 16
        for (int j = 0; j < kHD; ++j) {
            const float s = tile[j * CB + t];
            r = r + s * kn[j];
            p = p + s * qn[j];
        }
        const float vi = vp[h * kHD + c0 + t];
        const float delta = beta * (vi - decay * r);
        const float o = 0.0625f * (decay * p + alpha * delta);
        dl[t] = delta;
        attn[h * kHD + c0 + t] = R<C>(o);
    }
    __syncthreads();

    // Update pass: S' = decay * S + k (x) delta.
    if constexpr (C == kRef) {
        constexpr int PER_ROW = CB / 8;
        uint16_t *S = reinterpret_cast<uint16_t *>(state);
#pragma unroll
        for (int i = 0; i < (kHD * PER_ROW) / kT; ++i) {
            const int u = t + kT * i, row = u / PER_ROW, c8 = u - row * PER_ROW;
            const float kj = kn[row];
            uint32_t packed[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int col = c8 * 8 + 2 * e;
                const float n0 = decay * tile[row * CB + col] + kj * dl[col];
                const float n1 = decay * tile[row * CB + col + 1] + kj * dl[col + 1];
                packed[e] = (f2u(rne_bf16(n0)) >> 16) | (f2u(rne_bf16(n1)) & 0xffff0000u);
            }
            u32x4 v;
            v.x = packed[0]; v.y = packed[1]; v.z = packed[2]; v.w = packed[3];
            *reinterpret_cast<u32x4 *>(S + sbase + (size_t)row * kHD + c8 * 8) = v;
        }
    } else {
        constexpr int PER_ROW = CB / 4;
        float *S = reinterpret_cast<float *>(state);
#pragma unroll
        for (int i = 0; i < (kHD * PER_ROW) / kT; ++i) {
            const int u = t + kT * i, row = u / PER_ROW, c4 = u - row * PER_ROW;
            const float kj = kn[row];
            const f32x4 old = *reinterpret_cast<const f32x4 *>(tile + row * CB + c4 * 4);
            f32x4 nv;
            nv.x = decay * old.x + kj * dl[c4 * 4 + 0];
            nv.y = decay * old.y + kj * dl[c4 * 4 + 1];
            nv.z = decay * old.z + kj * dl[c4 * 4 + 2];
            nv.w = decay * old.w + kj * dl[c4 * 4 + 3];
            *reinterpret_cast<f32x4 *>(S + sbase + (size_t)row * kHD + c4 * 4) = nv;
        }
    }

    if (!do_onorm) return;
    // Output RMSNorm * gate for the head, by its last column block.
    if (!last_block_arrives(cnt + h, gridDim.x, &flag)) return;
    const float av = coherent_load(attn + h * kHD + t);
    if (t < kHD / 16) {
        float s = 0.0f;
#pragma unroll
        for (int kk = 0; kk < 16; ++kk) {
            const float v = coherent_load(attn + h * kHD + 16 * t + kk);
            s += v * v;
        }
        tile[t] = s;
    }
    __syncthreads();
    float sum = 0.0f;
    for (int i = 0; i < kHD / 16; ++i) sum += tile[i];
    const float scale = 1.0f / __builtin_sqrtf(sum / (float)kHD + eps);
    const float gv = gate[h * kHD + t];
    const float normalized = av * scale * onorm_w[t];
    og[h * kHD + t] = R<C>(normalized * gv * sigmoid_ref(gv));
}

// GEMV into a residual add + RMSNorm (o_proj, down).
template <int C, int K, int RB>
__global__ __launch_bounds__(kT) void k_gemv_res(const void *__restrict__ W,
                                                 const float *__restrict__ x, WInfo wi,
                                                 float *__restrict__ ybuf,
                                                 const float *__restrict__ res_in,
                                                 float *__restrict__ res_out,
                                                 const float *__restrict__ norm_w,
                                                 float *__restrict__ xn_out,
                                                 unsigned *__restrict__ cnt, float eps) {
    __shared__ __attribute__((aligned(16))) float xs[K];
    __shared__ __attribute__((aligned(16))) float part[RB * Hb<K>::HBP > kH / 16 ? RB * Hb<K>::HBP : kH / 16];
    __shared__ float red[4];
    __shared__ int redi[4];
    __shared__ int flag;
    static_assert(K >= kH, "the LDS x copy is reused for the residual");
    const float y = gemv_block<K, RB, C>(W, x, wi, xs, part, red, redi);
    const int lane = threadIdx.x;
    if (lane < 64 && (lane & 3) == 0 && (lane >> 2) < RB)
        ybuf[blockIdx.x * RB + (lane >> 2)] = R<C>(y);
    if (!last_block_arrives(cnt, gridDim.x, &flag)) return;
    for (int i = threadIdx.x; i < kH; i += kT) {
        const float xr = R<C>(res_in[i] + coherent_load(ybuf + i));
        res_out[i] = xr;
        xs[i] = xr;
    }
    __syncthreads();
    block_rmsnorm_h<C>(xs, norm_w, xn_out, eps, part);
}

// gate/up GEMV with rows interleaved in blocks of 4 + 4, SwiGLU epilogue.
template <int C>
__global__ __launch_bounds__(kT) void k_gu(const void *__restrict__ W, const float *__restrict__ x,
                                           WInfo wi, float *__restrict__ hout) {
    constexpr int RB = kRbGu;
    __shared__ __attribute__((aligned(16))) float xs[kH];
    __shared__ __attribute__((aligned(16))) float part[RB * Hb<kH>::HBP];
    __shared__ float red[4];
    __shared__ int redi[4];
    const float y = gemv_block<kH, RB, C>(W, x, wi, xs, part, red, redi);
    if (threadIdx.x < 64) {
        const float yu = __shfl_down(y, 4 * (RB / 2));
        const int lane = threadIdx.x;
        if ((lane & 3) == 0 && (lane >> 2) < RB / 2) {
            const float g = R<C>(y), u = R<C>(yu);
            hout[blockIdx.x * (RB / 2) + (lane >> 2)] = R<C>(silu_ref(g) * u);
        }
    }
}

// LM head: FP32 logits (not rounded) and the argmax (strict '>', lowest
// index on ties, running best from -FLT_MAX at index 0).
template <int C>
__global__ __launch_bounds__(kT) void k_lm(const void *__restrict__ W, const float *__restrict__ x,
                                           WInfo wi, float *__restrict__ logits,
                                           float *__restrict__ part_val, int *__restrict__ part_idx,
                                           unsigned *__restrict__ cnt, int *__restrict__ tok_out,
                                           float *__restrict__ ws_token) {
    constexpr int RB = kRbLm;
    __shared__ __attribute__((aligned(16))) float xs[kH];
    __shared__ __attribute__((aligned(16))) float part[RB * Hb<kH>::HBP];
    __shared__ float red[4];
    __shared__ int redi[4];
    __shared__ int flag;
    __shared__ float bv[4];
    __shared__ int bi[4];
    const float y = gemv_block<kH, RB, C>(W, x, wi, xs, part, red, redi);
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        const int row0 = blockIdx.x * RB;
        if ((lane & 3) == 0 && (lane >> 2) < RB) logits[row0 + (lane >> 2)] = y;
        float best = -3.402823466e38f;
        int idx = 0;
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const float v = __shfl(y, 4 * r);
            if (v > best) {
                best = v;
                idx = row0 + r;
            }
        }
        if (lane == 0) {
            part_val[blockIdx.x] = best;
            part_idx[blockIdx.x] = idx;
        }
    }
    if (!last_block_arrives(cnt, gridDim.x, &flag)) return;
    float best = -3.402823466e38f;
    int idx = 0;
    for (int i = threadIdx.x; i < (int)gridDim.x; i += kT) {
        const float v = coherent_load(part_val + i);
        const int id = __hip_atomic_load(part_idx + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (v > best) {
            best = v;
            idx = id;
        }
    }
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
        const float ov = __shfl_xor(best, m);
        const int oi = __shfl_xor(idx, m);
        if (ov > best || (ov == best && oi < idx)) {
            best = ov;
            idx = oi;
        }
    }
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    if (lane == 0) {
        bv[w] = best;
        bi[w] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int i = 1; i < 4; ++i) {
            if (bv[i] > best || (bv[i] == best && bi[i] < idx)) {
                best = bv[i];
                idx = bi[i];
            }
        }
        tok_out[0] = idx;
        ws_token[0] = (float)idx;
    }
}

// Plain GEMV: FP32 row results before any rounding point (test hook).
template <int C, int K, int RB>
__global__ __launch_bounds__(kT) void k_gemv_plain(const void *__restrict__ W,
                                                   const float *__restrict__ x, WInfo wi,
                                                   float *__restrict__ y_out) {
    __shared__ __attribute__((aligned(16))) float xs[K];
    __shared__ __attribute__((aligned(16))) float part[RB * Hb<K>::HBP];
    __shared__ float red[4];
    __shared__ int redi[4];
    const float y = gemv_block<K, RB, C>(W, x, wi, xs, part, red, redi);
    const int lane = threadIdx.x;
    if (lane < 64 && (lane & 3) == 0 && (lane >> 2) < RB) y_out[blockIdx.x * RB + (lane >> 2)] = y;
}

}  // namespace gdn

// ===================================================================== engine

using namespace gdn;

struct GDNEngine {
    int contract = 0;
    int layers = 0;
    int vocab = 0;
    float eps = 1e-6f;
    hipStream_t stream = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    // weights
    void *wmem = nullptr;
    void *w_qkvg[kMaxLayers] = {}, *w_o[kMaxLayers] = {}, *w_gu[kMaxLayers] = {},
         *w_down[kMaxLayers] = {};
    void *w_lm = nullptr, *w_emb = nullptr;
    WInfo i_qkvg[kMaxLayers] = {}, i_o[kMaxLayers] = {}, i_gu[kMaxLayers] = {},
          i_down[kMaxLayers] = {}, i_lm = {};
    float *aux = nullptr;  // [layers][kAuxLayer] + final_norm[kH]
    // workspace (GDN_WS_OFF_* layout) and activations
    float *ws = nullptr;
    float *act = nullptr;
    float *resid = nullptr, *resid_alt = nullptr, *xn = nullptr, *qkv = nullptr,
          *gate = nullptr, *ab = nullptr, *attn = nullptr, *og = nullptr, *ybuf = nullptr,
          *hbuf = nullptr, *lm_val = nullptr;
    int *lm_idx = nullptr;
    unsigned *counters = nullptr;
    int *tok_dev = nullptr;   // [0] in, [1] out
    int *tok_host = nullptr;  // pinned [0] in, [1] out
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    bool use_graph = true;
};

namespace {

size_t welem(int contract) { return contract == kFp32 ? 4 : 2; }

float *layer_aux(GDNEngine *e, int l) { return e->aux + (size_t)l * kAuxLayer; }
float *final_norm(GDNEngine *e) { return e->aux + (size_t)e->layers * kAuxLayer; }
unsigned *cnt_recur(GDNEngine *e, int l) { return e->counters + (size_t)l * 16; }
unsigned *cnt_o(GDNEngine *e, int l) { return e->counters + (size_t)l * 16 + 8; }
unsigned *cnt_down(GDNEngine *e, int l) { return e->counters + (size_t)l * 16 + 9; }
unsigned *cnt_lm(GDNEngine *e) { return e->counters + (size_t)e->layers * 16; }
float *layer_tails(GDNEngine *e, int l) {
    return e->ws + GDN_WS_OFF_HEAD_BUF + (size_t)l * 3 * kTailStripe;
}
void *layer_state(GDNEngine *e, int l) {
    const size_t off = (size_t)l * kNH * kHD * kHD;
    if (e->contract == kRef)
        return reinterpret_cast<uint16_t *>(e->ws + GDN_WS_OFF_REC_STATE) + off;
    return e->ws + GDN_WS_OFF_REC_STATE + off;
}

// Pack rows of BF16-exact FP32 words into the device matrix at `dst`.
struct Packer {
    int contract;
    std::vector<unsigned char> staging;
    float min_abs = INFINITY;
    int nonfinite = 0;
    size_t filled = 0;  // elements

    void begin(size_t elems) {
        staging.resize(elems * welem(contract));
        min_abs = INFINITY;
        nonfinite = 0;
        filled = 0;
    }
    void rows(const float *src, size_t n, bool daz = true) {
        float mn;
        int bad;
        if (contract == kFp32) {
            std::memcpy(staging.data() + filled * 4, src, n * 4);
            gdn_scan_fp32(src, n, &mn, &bad);
        } else {
            uint16_t *d = reinterpret_cast<uint16_t *>(staging.data()) + filled;
            if (daz) {
                gdn_pack_bf16_daz(src, d, n, &mn, &bad);
            } else {
                for (size_t i = 0; i < n; ++i) {
                    uint32_t b;
                    std::memcpy(&b, src + i, 4);
                    d[i] = (uint16_t)(b >> 16);
                }
                mn = INFINITY;
                bad = 0;
            }
        }
        if (mn < min_abs) min_abs = mn;
        nonfinite |= bad;
        filled += n;
    }
    int upload(void *dst) {
        GDN_HIP(hipMemcpy(dst, staging.data(), filled * welem(contract), hipMemcpyHostToDevice));
        return 0;
    }
    WInfo info() const { return WInfo{min_abs, nonfinite}; }
};

int check_shape(const GDNWeightHeader *c) {
    if (c->hidden_size != (uint32_t)kH || c->num_heads != (uint32_t)kNH ||
        c->num_v_heads != (uint32_t)kNH || c->head_dim != (uint32_t)kHD ||
        c->intermediate_size != (uint32_t)kI || c->conv_size != 4u) {
        gdn_error("gdn: the engine is specialised for hidden 2048, 8x256 heads, "
                  "intermediate 5632, conv 4");
        return -1;
    }
    if (c->num_layers < 1 || c->num_layers > (uint32_t)kMaxLayers) {
        gdn_error("gdn: num_layers must be 1..24");
        return -1;
    }
    if (c->vocab_size == 0 || (c->vocab_size % kRbLm) != 0) {
        gdn_error("gdn: vocab_size must be a positive multiple of 8");
        return -1;
    }
    return 0;
}

int upload_weights(GDNEngine *e, const GDNModel *m) {
    const size_t H = kH, I = kI, V = (size_t)e->vocab, L = (size_t)e->layers;
    const size_t per_layer = 4 * H * H + H * H + 2 * I * H + H * I;
    const size_t total = L * per_layer + 2 * V * H;
    const size_t es = welem(e->contract);
    GDN_HIP(hipMalloc(&e->wmem, total * es));
    char *p = static_cast<char *>(e->wmem);
    Packer pk{e->contract, {}};
    for (size_t l = 0; l < L; ++l) {
        const GDNLayerWeights &w = m->layers[l];
        pk.begin(4 * H * H);
        pk.rows(w.q_proj, H * H);
        pk.rows(w.k_proj, H * H);
        pk.rows(w.v_proj, H * H);
        pk.rows(w.g_proj, H * H);
        e->w_qkvg[l] = p;
        e->i_qkvg[l] = pk.info();
        if (pk.upload(p)) return -1;
        p += 4 * H * H * es;

        pk.begin(H * H);
        pk.rows(w.o_proj, H * H);
        e->w_o[l] = p;
        e->i_o[l] = pk.info();
        if (pk.upload(p)) return -1;
        p += H * H * es;

        pk.begin(2 * I * H);
        for (size_t blk = 0; blk < I / (kRbGu / 2); ++blk) {
            pk.rows(w.mlp_gate_proj + blk * (kRbGu / 2) * H, (kRbGu / 2) * H);
            pk.rows(w.mlp_up_proj + blk * (kRbGu / 2) * H, (kRbGu / 2) * H);
        }
        e->w_gu[l] = p;
        e->i_gu[l] = pk.info();
        if (pk.upload(p)) return -1;
        p += 2 * I * H * es;

        pk.begin(H * I);
        pk.rows(w.mlp_down_proj, H * I);
        e->w_down[l] = p;
        e->i_down[l] = pk.info();
        if (pk.upload(p)) return -1;
        p += H * I * es;
    }
    pk.begin(V * H);
    pk.rows(m->lm_head, V * H);
    e->w_lm = p;
    e->i_lm = pk.info();
    if (pk.upload(p)) return -1;
    p += V * H * es;

    pk.begin(V * H);
    pk.rows(m->embeddings, V * H, /*daz=*/false);
    e->w_emb = p;
    if (pk.upload(p)) return -1;
    p += V * H * es;
    std::vector<unsigned char>().swap(pk.staging);

    // Small FP32 weights.
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
    GDN_HIP(hipDeviceSynchronize());
    return 0;
}

int alloc_buffers(GDNEngine *e) {
    GDN_HIP(hipMalloc(&e->ws, (size_t)GDN_WS_FLOATS * 4));
    GDN_HIP(hipMemset(e->ws, 0, (size_t)GDN_WS_FLOATS * 4));
    const size_t nblk_lm = (size_t)e->vocab / kRbLm;
    const size_t act_floats = 2 * kH + kI + 3 * kH + kH + 16 + kH + kH + kH + kI + nblk_lm;
    GDN_HIP(hipMalloc(&e->act, act_floats * 4));
    GDN_HIP(hipMemset(e->act, 0, act_floats * 4));
    float *p = e->act;
    e->resid = p; p += kH;
    e->resid_alt = p; p += kH;
    e->xn = p; p += kI;
    e->qkv = p; p += 3 * kH;
    e->gate = p; p += kH;
    e->ab = p; p += 16;
    e->attn = p; p += kH;
    e->og = p; p += kH;
    e->ybuf = p; p += kH;
    e->hbuf = p; p += kI;
    e->lm_val = p; p += nblk_lm;
    GDN_HIP(hipMalloc(&e->lm_idx, nblk_lm * sizeof(int)));
    const size_t ncnt = (size_t)(e->layers + 1) * 16;
    GDN_HIP(hipMalloc(&e->counters, ncnt * sizeof(unsigned)));
    GDN_HIP(hipMemset(e->counters, 0, ncnt * sizeof(unsigned)));
    GDN_HIP(hipMalloc(&e->tok_dev, 2 * sizeof(int)));
    GDN_HIP(hipMemset(e->tok_dev, 0, 2 * sizeof(int)));
    GDN_HIP(hipHostMalloc(&e->tok_host, 2 * sizeof(int), hipHostMallocDefault));
    e->tok_host[0] = e->tok_host[1] = 0;
    GDN_HIP(hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking));
    GDN_HIP(hipEventCreate(&e->ev0));
    GDN_HIP(hipEventCreate(&e->ev1));
    return 0;
}

template <int C>
void enqueue_layer(GDNEngine *e, int l, hipStream_t s) {
    float *aux = layer_aux(e, l);
    const float *next_norm = (l + 1 < e->layers) ? layer_aux(e, l + 1) + kAuxAttnNorm : final_norm(e);
    hipLaunchKernelGGL((k_qkvg<C, kRbQkvg>), dim3(4 * kH / kRbQkvg + 1), dim3(kT), 0, s,
                       e->w_qkvg[l], e->xn, e->i_qkvg[l], aux, layer_tails(e, l), e->qkv, e->gate,
                       e->ab);
    hipLaunchKernelGGL((k_recur<C, kCB>), dim3(kHD / kCB, kNH), dim3(kT), 0, s, e->qkv,
                       e->qkv + kH, e->qkv + 2 * kH, e->ab, e->ab + kNH, aux + kAuxALog,
                       aux + kAuxDtBias, layer_state(e, l), e->attn, e->gate, aux + kAuxONorm,
                       e->og, cnt_recur(e, l), e->eps, 1);
    hipLaunchKernelGGL((k_gemv_res<C, kH, kRbO>), dim3(kH / kRbO), dim3(kT), 0, s, e->w_o[l],
                       e->og, e->i_o[l], e->ybuf, e->resid, e->resid_alt, aux + kAuxMlpNorm,
                       e->xn, cnt_o(e, l), e->eps);
    hipLaunchKernelGGL((k_gu<C>), dim3(2 * kI / kRbGu), dim3(kT), 0, s, e->w_gu[l], e->xn,
                       e->i_gu[l], e->hbuf);
    hipLaunchKernelGGL((k_gemv_res<C, kI, kRbDown>), dim3(kH / kRbDown), dim3(kT), 0, s,
                       e->w_down[l], e->hbuf, e->i_down[l], e->ybuf, e->resid_alt, e->resid,
                       next_norm, e->xn, cnt_down(e, l), e->eps);
}

template <int C>
void enqueue_step_t(GDNEngine *e, hipStream_t s) {
    hipLaunchKernelGGL((k_embed<C>), dim3(1), dim3(kT), 0, s, e->tok_dev, e->vocab, e->w_emb,
                       (const float *)nullptr, e->ws + GDN_WS_OFF_X, e->resid,
                       layer_aux(e, 0) + kAuxAttnNorm, e->xn, e->eps);
    for (int l = 0; l < e->layers; ++l) enqueue_layer<C>(e, l, s);
    hipLaunchKernelGGL((k_lm<C>), dim3(e->vocab / kRbLm), dim3(kT), 0, s, e->w_lm, e->xn, e->i_lm,
                       e->ws + GDN_WS_OFF_LOGITS, e->lm_val, e->lm_idx, cnt_lm(e), e->tok_dev + 1,
                       e->ws + GDN_WS_OFF_X_NORM);
}

void enqueue_step(GDNEngine *e, hipStream_t s) {
    switch (e->contract) {
    case kRef: enqueue_step_t<kRef>(e, s); break;
    case kBf16w: enqueue_step_t<kBf16w>(e, s); break;
    default: enqueue_step_t<kFp32>(e, s); break;
    }
}

int ensure_graph(GDNEngine *e) {
    if (e->exec) return 0;
    GDN_HIP(hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal));
    enqueue_step(e, e->stream);
    GDN_HIP(hipStreamEndCapture(e->stream, &e->graph));
    GDN_HIP(hipGraphInstantiate(&e->exec, e->graph, nullptr, nullptr, 0));
    return 0;
}

// Token in (host) -> kernels -> token out (host).  Times when asked.
int run_step(GDNEngine *e, int32_t token, int32_t *tok_out, float *inner_ms) {
    if (e->use_graph && ensure_graph(e) != 0) return -1;
    e->tok_host[0] = token;
    GDN_HIP(hipMemcpyAsync(e->tok_dev, e->tok_host, sizeof(int), hipMemcpyHostToDevice, e->stream));
    if (inner_ms) GDN_HIP(hipEventRecord(e->ev0, e->stream));
    if (e->use_graph) {
        GDN_HIP(hipGraphLaunch(e->exec, e->stream));
    } else {
        enqueue_step(e, e->stream);
        GDN_HIP(hipGetLastError());
    }
    if (inner_ms) GDN_HIP(hipEventRecord(e->ev1, e->stream));
    GDN_HIP(hipMemcpyAsync(e->tok_host + 1, e->tok_dev + 1, sizeof(int), hipMemcpyDeviceToHost,
                           e->stream));
    GDN_HIP(hipStreamSynchronize(e->stream));
    if (tok_out) *tok_out = e->tok_host[1];
    if (inner_ms) GDN_HIP(hipEventElapsedTime(inner_ms, e->ev0, e->ev1));
    return 0;
}

void destroy_engine(GDNEngine *e) {
    if (!e) return;
    if (e->exec) (void)hipGraphExecDestroy(e->exec);
    if (e->graph) (void)hipGraphDestroy(e->graph);
    if (e->ev0) (void)hipEventDestroy(e->ev0);
    if (e->ev1) (void)hipEventDestroy(e->ev1);
    if (e->stream) (void)hipStreamDestroy(e->stream);
    (void)hipFree(e->wmem);
    (void)hipFree(e->aux);
    (void)hipFree(e->ws);
    (void)hipFree(e->act);
    (void)hipFree(e->lm_idx);
    (void)hipFree(e->counters);
    (void)hipFree(e->tok_dev);
    if (e->tok_host) (void)hipHostFree(e->tok_host);
    delete e;
}

bool bf16_exact(float v) {
    uint32_t b;
    std::memcpy(&b, &v, 4);
    return (b & 0xffffu) == 0;
}

}  // namespace

// ================================================================== C ABI

extern "C" {

int gdn_run_state_init_contract(GDNRunState *state, const GDNModel *model, uint32_t max_tokens,
                                int contract) {
    std::memset(state, 0, sizeof(*state));
    if (max_tokens == 0 || max_tokens > model->config.max_seq_len) {
        gdn_error("invalid max_tokens for run state");
        return -1;
    }
    if (contract < kRef || contract > kFp32) {
        gdn_error("gdn: unknown contract");
        return -1;
    }
    if (check_shape(&model->config) != 0) return -1;
    if (contract != kFp32 && gdn_validate_bf16_exact_weights(model->weight_data, &model->config) != 0) {
        gdn_error("gdn: BF16 contracts need a BF16-exact checkpoint");
        return -1;
    }
    GDNEngine *e = new GDNEngine();
    e->contract = contract;
    e->layers = (int)model->config.num_layers;
    e->vocab = (int)model->config.vocab_size;
    e->eps = model->config.norm_eps;
    if (alloc_buffers(e) != 0 || upload_weights(e, model) != 0) {
        destroy_engine(e);
        return -1;
    }
    state->engine = e;
    state->workspace = e->ws;
    state->x = e->ws + GDN_WS_OFF_X;
    state->recurrent_state = e->ws + GDN_WS_OFF_REC_STATE;
    state->head_buffer = e->ws + GDN_WS_OFF_HEAD_BUF;
    return 0;
}

int gdn_run_state_init(GDNRunState *state, const GDNModel *model, uint32_t max_tokens) {
    return gdn_run_state_init_contract(state, model, max_tokens, kRef);
}

void gdn_run_state_free(GDNRunState *state) {
    destroy_engine(state->engine);
    std::memset(state, 0, sizeof(*state));
}

int gdn_get_contract(const GDNRunState *state) {
    return state->engine ? state->engine->contract : -1;
}

int gdn_set_graph_mode(GDNRunState *state, int use_graph) {
    if (!state->engine) return -1;
    state->engine->use_graph = use_graph != 0;
    return 0;
}

int gdn_decode_step_host(const GDNModel *model, GDNRunState *state, const int32_t *token) {
    if (*token < 0 || (uint32_t)*token >= model->config.vocab_size) {
        gdn_error("token id out of range");
        return -1;
    }
    if (!state->engine) {
        gdn_error("gdn: run state not initialised");
        return -1;
    }
    return run_step(state->engine, *token, nullptr, nullptr);
}

int gdn_read_token(const GDNRunState *state, int32_t *token) {
    GDN_HIP(hipMemcpy(token, state->engine->tok_dev + 1, sizeof(int32_t), hipMemcpyDeviceToHost));
    return 0;
}

int gdn_read_logits(const GDNRunState *state, float *logits, size_t count) {
    if (count > (size_t)state->engine->vocab) return -1;
    GDN_HIP(hipMemcpy(logits, state->engine->ws + GDN_WS_OFF_LOGITS, count * 4, hipMemcpyDeviceToHost));
    return 0;
}

int gdn_read_final_hidden(const GDNRunState *state, float *hidden, size_t count) {
    if (count > (size_t)kH) return -1;
    GDN_HIP(hipMemcpy(hidden, state->engine->xn, count * 4, hipMemcpyDeviceToHost));
    return 0;
}

int gdn_load_recurrent_state(GDNRunState *state, const float *rec, size_t floats) {
    GDNEngine *e = state->engine;
    const size_t n = (size_t)e->layers * kNH * kHD * kHD;
    if (floats != n) {
        gdn_error("recurrent state size does not match the model");
        return -1;
    }
    if (e->contract == kRef) {
        std::vector<uint16_t> b(n);
        for (size_t i = 0; i < n; ++i) {
            if (!bf16_exact(rec[i])) {
                std::fprintf(stderr, "gdn: recurrent state %zu is not BF16-exact\n", i);
                return -1;
            }
            uint32_t u;
            std::memcpy(&u, rec + i, 4);
            b[i] = (uint16_t)(u >> 16);
        }
        GDN_HIP(hipMemcpy(layer_state(e, 0), b.data(), n * 2, hipMemcpyHostToDevice));
    } else {
        GDN_HIP(hipMemcpy(layer_state(e, 0), rec, n * 4, hipMemcpyHostToDevice));
    }
    GDN_HIP(hipDeviceSynchronize());
    return 0;
}

int gdn_save_recurrent_state(const GDNRunState *state, float *rec, size_t floats) {
    GDNEngine *e = state->engine;
    const size_t n = (size_t)e->layers * kNH * kHD * kHD;
    if (floats != n) return -1;
    if (e->contract == kRef) {
        std::vector<uint16_t> b(n);
        GDN_HIP(hipMemcpy(b.data(), layer_state(e, 0), n * 2, hipMemcpyDeviceToHost));
        for (size_t i = 0; i < n; ++i) {
            const uint32_t u = (uint32_t)b[i] << 16;
            std::memcpy(rec + i, &u, 4);
        }
    } else {
        GDN_HIP(hipMemcpy(rec, layer_state(e, 0), n * 4, hipMemcpyDeviceToHost));
    }
    return 0;
}

// .gdnstate conv section [L][q,k,v][W-1][H] <-> per-stripe device tails.
int gdn_load_conv_tails(GDNRunState *state, const float *conv, size_t floats) {
    GDNEngine *e = state->engine;
    const size_t stripes = (size_t)e->layers * 3, per = 3 * (size_t)kH;
    if (floats != stripes * per) {
        gdn_error("convolution-tail size does not match the model");
        return -1;
    }
    std::vector<float> img(stripes * kTailStripe, 0.0f);
    for (size_t s = 0; s < stripes; ++s) {
        float *dst = img.data() + s * kTailStripe;
        const float *src = conv + s * per;
        if (e->contract == kFp32) {
            std::memcpy(dst, src, per * 4);
        } else {
            uint16_t *d16 = reinterpret_cast<uint16_t *>(dst);
            for (size_t i = 0; i < per; ++i) {
                if (!bf16_exact(src[i])) {
                    std::fprintf(stderr, "gdn: convolution tail %zu is not BF16-exact\n", s * per + i);
                    return -1;
                }
                uint32_t u;
                std::memcpy(&u, src + i, 4);
                d16[i] = (uint16_t)(u >> 16);
            }
        }
    }
    GDN_HIP(hipMemcpy(e->ws + GDN_WS_OFF_HEAD_BUF, img.data(), img.size() * 4, hipMemcpyHostToDevice));
    GDN_HIP(hipDeviceSynchronize());
    return 0;
}

int gdn_save_conv_tails(const GDNRunState *state, float *conv, size_t floats) {
    GDNEngine *e = state->engine;
    const size_t stripes = (size_t)e->layers * 3, per = 3 * (size_t)kH;
    if (floats != stripes * per) return -1;
    std::vector<float> img(stripes * kTailStripe);
    GDN_HIP(hipMemcpy(img.data(), e->ws + GDN_WS_OFF_HEAD_BUF, img.size() * 4, hipMemcpyDeviceToHost));
    for (size_t s = 0; s < stripes; ++s) {
        const float *src = img.data() + s * kTailStripe;
        float *dst = conv + s * per;
        if (e->contract == kFp32) {
            std::memcpy(dst, src, per * 4);
        } else {
            const uint16_t *s16 = reinterpret_cast<const uint16_t *>(src);
            for (size_t i = 0; i < per; ++i) {
                const uint32_t u = (uint32_t)s16[i] << 16;
                std::memcpy(dst + i, &u, 4);
            }
        }
    }
    return 0;
}

int gdn_run_teacher_forced(GDNRunState *state, const int32_t *tokens, uint32_t n_tokens,
                           uint32_t n_steps, int32_t *argmax_out, float *inner_ms,
                           float *outer_ms) {
    GDNEngine *e = state->engine;
    if (!e || n_tokens == 0) return -1;
    for (uint32_t i = 0; i < n_tokens; ++i) {
        if (tokens[i] < 0 || tokens[i] >= e->vocab) {
            gdn_error("token id out of range");
            return -1;
        }
    }
    if (e->use_graph && ensure_graph(e) != 0) return -1;
    for (uint32_t s = 0; s < n_steps; ++s) {
        const auto t0 = std::chrono::steady_clock::now();
        int32_t out = 0;
        float inner = 0.0f;
        if (run_step(e, tokens[s % n_tokens], &out, inner_ms ? &inner : nullptr) != 0) return -1;
        const auto t1 = std::chrono::steady_clock::now();
        if (argmax_out) argmax_out[s] = out;
        if (inner_ms) inner_ms[s] = inner;
        if (outer_ms) outer_ms[s] = std::chrono::duration<float, std::milli>(t1 - t0).count();
    }
    return 0;
}

// ---------------------------------------------------------------- test hooks

int gdn_test_gemv(int contract, const float *W, const float *x, uint32_t M, uint32_t K, float *y) {
    if ((K != (uint32_t)kH && K != (uint32_t)kI) || M == 0 || (M % kRbTest) != 0) {
        gdn_error("gdn_test_gemv: K must be 2048 or 5632 and M a multiple of 8");
        return -1;
    }
    Packer pk{contract, {}};
    pk.begin((size_t)M * K);
    pk.rows(W, (size_t)M * K);
    void *dW = nullptr;
    float *dx = nullptr, *dy = nullptr;
    GDN_HIP(hipMalloc(&dW, (size_t)M * K * welem(contract)));
    GDN_HIP(hipMalloc(&dx, (size_t)K * 4));
    GDN_HIP(hipMalloc(&dy, (size_t)M * 4));
    if (pk.upload(dW)) return -1;
    GDN_HIP(hipMemcpy(dx, x, (size_t)K * 4, hipMemcpyHostToDevice));
    const WInfo wi = pk.info();
    const dim3 grid(M / kRbTest), block(kT);
#define GDN_PLAIN(CC, KK) hipLaunchKernelGGL((k_gemv_plain<CC, KK, kRbTest>), grid, block, 0, 0, dW, dx, wi, dy)
    if (K == (uint32_t)kH) {
        if (contract == kFp32) GDN_PLAIN(kFp32, kH);
        else GDN_PLAIN(kRef, kH);
    } else {
        if (contract == kFp32) GDN_PLAIN(kFp32, kI);
        else GDN_PLAIN(kRef, kI);
    }
#undef GDN_PLAIN
    GDN_HIP(hipGetLastError());
    GDN_HIP(hipMemcpy(y, dy, (size_t)M * 4, hipMemcpyDeviceToHost));
    GDN_HIP(hipFree(dW));
    GDN_HIP(hipFree(dx));
    GDN_HIP(hipFree(dy));
    return 0;
}

int gdn_test_recurrence(int contract, uint32_t n_heads, uint32_t n_steps, const float *q,
                        const float *k, const float *v, const float *a, const float *b,
                        const float *a_log, const float *dt_bias, float *S, float *o) {
    if (n_heads == 0 || n_heads > 65535 || contract < kRef || contract > kFp32) return -1;
    const size_t nv = (size_t)n_steps * n_heads * kHD, ns = (size_t)n_steps * n_heads;
    const size_t nstate = (size_t)n_heads * kHD * kHD;
    float *dq, *dk, *dv, *da, *db, *dal, *ddt, *dout;
    void *dS;
    GDN_HIP(hipMalloc(&dq, nv * 4));
    GDN_HIP(hipMalloc(&dk, nv * 4));
    GDN_HIP(hipMalloc(&dv, nv * 4));
    GDN_HIP(hipMalloc(&dout, nv * 4));
    GDN_HIP(hipMalloc(&da, ns * 4));
    GDN_HIP(hipMalloc(&db, ns * 4));
    GDN_HIP(hipMalloc(&dal, ns * 4));
    GDN_HIP(hipMalloc(&ddt, ns * 4));
    GDN_HIP(hipMalloc(&dS, nstate * 4));
    GDN_HIP(hipMemcpy(dq, q, nv * 4, hipMemcpyHostToDevice));
    GDN_HIP(hipMemcpy(dk, k, nv * 4, hipMemcpyHostToDevice));
    GDN_HIP(hipMemcpy(dv, v, nv * 4, hipMemcpyHostToDevice));
    GDN_HIP(hipMemcpy(da, a, ns * 4, hipMemcpyHostToDevice));
    GDN_HIP(hipMemcpy(db, b, ns * 4, hipMemcpyHostToDevice));
    GDN_HIP(hipMemcpy(dal, a_log, ns * 4, hipMemcpyHostToDevice));
    GDN_HIP(hipMemcpy(ddt, dt_bias, ns * 4, hipMemcpyHostToDevice));
    if (contract == kRef) {
        std::vector<uint16_t> sb(nstate);
        for (size_t i = 0; i < nstate; ++i) {
            uint32_t u;
            std::memcpy(&u, S + i, 4);
            sb[i] = (uint16_t)(u >> 16);
        }
        GDN_HIP(hipMemcpy(dS, sb.data(), nstate * 2, hipMemcpyHostToDevice));
    } else {
        GDN_HIP(hipMemcpy(dS, S, nstate * 4, hipMemcpyHostToDevice));
    }
    const dim3 grid(kHD / kCB, n_heads), block(kT);
    for (uint32_t s = 0; s < n_steps; ++s) {
        const size_t ov = (size_t)s * n_heads * kHD, os = (size_t)s * n_heads;
#define GDN_REC(CC)                                                                           \
    hipLaunchKernelGGL((k_recur<CC, kCB>), grid, block, 0, 0, dq + ov, dk + ov, dv + ov,       \
                       da + os, db + os, dal + os, ddt + os, dS, dout + ov, (const float *)nullptr, \
                       (const float *)nullptr, (float *)nullptr, (unsigned *)nullptr, 0.0f, 0)
        if (contract == kRef) GDN_REC(kRef);
        else if (contract == kBf16w) GDN_REC(kBf16w);
        else GDN_REC(kFp32);
#undef GDN_REC
    }
    GDN_HIP(hipGetLastError());
    GDN_HIP(hipDeviceSynchronize());
    GDN_HIP(hipMemcpy(o, dout, nv * 4, hipMemcpyDeviceToHost));
    if (contract == kRef) {
        std::vector<uint16_t> sb(nstate);
        GDN_HIP(hipMemcpy(sb.data(), dS, nstate * 2, hipMemcpyDeviceToHost));
        for (size_t i = 0; i < nstate; ++i) {
            const uint32_t u = (uint32_t)sb[i] << 16;
            std::memcpy(S + i, &u, 4);
        }
    } else {
        GDN_HIP(hipMemcpy(S, dS, nstate * 4, hipMemcpyDeviceToHost));
    }
    float *bufs[] = {dq, dk, dv, da, db, dal, ddt, dout};
    for (float *p : bufs) GDN_HIP(hipFree(p));
    GDN_HIP(hipFree(dS));
    return 0;
}

// Layer `layer` of the run state for n_steps residual inputs x_in[s] (H
// floats each); x_out[s] receives the layer's residual output.
int gdn_test_layer(GDNRunState *state, uint32_t layer, uint32_t n_steps, const float *x_in,
                   float *x_out) {
    GDNEngine *e = state->engine;
    if (!e || layer >= (uint32_t)e->layers) return -1;
    float *din;
    GDN_HIP(hipMalloc(&din, (size_t)kH * 4));
    for (uint32_t s = 0; s < n_steps; ++s) {
        GDN_HIP(hipMemcpyAsync(din, x_in + (size_t)s * kH, (size_t)kH * 4, hipMemcpyHostToDevice,
                               e->stream));
        const float *norm0 = layer_aux(e, (int)layer) + kAuxAttnNorm;
#define GDN_LAYER(CC)                                                                         \
    do {                                                                                      \
        hipLaunchKernelGGL((k_embed<CC>), dim3(1), dim3(kT), 0, e->stream, e->tok_dev, e->vocab, \
                           e->w_emb, din, e->ws + GDN_WS_OFF_X, e->resid, norm0, e->xn, e->eps); \
        enqueue_layer<CC>(e, (int)layer, e->stream);                                          \
    } while (0)
        if (e->contract == kRef) GDN_LAYER(kRef);
        else if (e->contract == kBf16w) GDN_LAYER(kBf16w);
        else GDN_LAYER(kFp32);
#undef GDN_LAYER
        GDN_HIP(hipGetLastError());
        GDN_HIP(hipMemcpyAsync(x_out + (size_t)s * kH, e->resid, (size_t)kH * 4,
                               hipMemcpyDeviceToHost, e->stream));
        GDN_HIP(hipStreamSynchronize(e->stream));
    }
    GDN_HIP(hipFree(din));
    return 0;
}

}  // extern "C"

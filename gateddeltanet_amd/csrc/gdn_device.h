// gdn_device.h -- constants, vector types and scalar device arithmetic
// shared by the batch-1 engine (gdn_engine.hip) and the multi-stream engine
// (gdn_batch.hip) of libgdn_amd.so.  Not part of the ABI.
#ifndef GDN_DEVICE_H
#define GDN_DEVICE_H

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>

#include "gdn_amd.h"
#include "gdn_libm.h"

// Host side: return -1 from the enclosing function when a HIP call fails.
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
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------- scalar math

// Phase stamps of the instrumented kernels (ST: compiled only into their
// own instantiations, so the uninstrumented kernels carry no trace of
// them): thread 0 of workgroup wg stores the 100 MHz real-time counter in
// slot k of its kStampSlots.  Slots: 0 start, 1 input ready, 2 products
// done, 3 end.
constexpr int kStampSlots = 4;
template <bool ST>
__device__ __forceinline__ void phase_stamp(uint64_t *stamps, int wg, int k) {
    if constexpr (ST) {
        if (threadIdx.x == 0) stamps[wg * kStampSlots + k] = __builtin_amdgcn_s_memrealtime();
    }
}

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
// The BF16 bits of a BF16-valued float (its top half).
__device__ __forceinline__ uint16_t bf16_hi(float x) { return (uint16_t)(f2u(x) >> 16); }

// expf and log1pf as the reference's C library evaluates them (glibc 2.35,
// gdn_libm.h): the engine's transcendentals equal the reference's bit for bit.
// Tab: where expf's 32-entry table is read (gdn_libm::Exp2Const, or Exp2Lds:
// a workgroup's copy in LDS, filled by fill_exp2_lds).
using Exp2Const = gdn_libm::Exp2Const;
struct Exp2Lds {
    const uint64_t *t;
    __device__ __forceinline__ uint64_t operator()(int i) const { return t[i]; }
};
// Threads 0..31: entry t of the table.  Load early (load()), store late
// (store(), before a barrier that precedes the first use).
struct Exp2Fill {
    uint64_t v = 0;
    __device__ __forceinline__ void load() {
        if (threadIdx.x < 32) v = gdn_libm::exp2_table((int)threadIdx.x);
    }
    __device__ __forceinline__ void store(uint64_t *lds) const {
        if (threadIdx.x < 32) lds[threadIdx.x] = v;
    }
};
// The same table written into LDS by threads 0..31 from immediates: no
// memory load, so no wait on the vector memory counter (which, in a GEMV's
// prologue waves, also counts their stores and could not be counted
// exactly across the prologue's branches).
__device__ __forceinline__ void fill_exp2_lds_imm(uint64_t *lds) {
    if (threadIdx.x < 32) {
        uint64_t v = 0;
#pragma unroll
        for (int i = 0; i < 32; ++i)
            if (threadIdx.x == (unsigned)i) v = gdn_libm::exp2_table(i);
        lds[threadIdx.x] = v;
    }
}

template <class Tab = Exp2Const>
__device__ __forceinline__ float exp_ref(float x, const Tab &tab = Tab()) { return gdn_libm::gdn_expf_t(x, tab); }
__device__ __forceinline__ float log1p_ref(float x) { return gdn_libm::gdn_log1pf(x); }

// gdn_sigmoid / gdn_silu / gdn_softplus, gdn_model.cpp:1307-1330.
template <class Tab = Exp2Const>
__device__ __forceinline__ float sigmoid_ref(float x, const Tab &tab = Tab()) {
    if (x >= 0.0f) {
        const float z = exp_ref(-x, tab);
        return 1.0f / (1.0f + z);
    }
    const float z = exp_ref(x, tab);
    return z / (1.0f + z);
}
template <class Tab = Exp2Const>
__device__ __forceinline__ float silu_ref(float x, const Tab &tab = Tab()) { return x * sigmoid_ref(x, tab); }
template <class Tab = Exp2Const>
__device__ __forceinline__ float softplus_ref(float x, const Tab &tab = Tab()) {
    if (x > 20.0f) return x;
    if (x < -20.0f) return exp_ref(x, tab);
    return log1p_ref(exp_ref(x, tab));
}

// Balanced pairwise sum of 16 contiguous values (gemv32_tree16).
__device__ __forceinline__ float tree16(const float *p) {
    const float s0 = p[0] + p[1], s1 = p[2] + p[3], s2 = p[4] + p[5], s3 = p[6] + p[7];
    const float s4 = p[8] + p[9], s5 = p[10] + p[11], s6 = p[12] + p[13], s7 = p[14] + p[15];
    const float a0 = s0 + s1, a1 = s2 + s3, a2 = s4 + s5, a3 = s6 + s7;
    const float b0 = a0 + a1, b1 = a2 + a3;
    return b0 + b1;
}

// Reduction of a wave64's 64 values by a commutative operation, left in
// every lane, in the pairing of an XOR butterfly: level m combines the
// partials of partner blocks of m lanes.  After each level every lane of a
// block holds the same value, so any lane of the partner block serves: quad
// permutes for m = 1, 2, the half-row and row mirrors for m = 4, 8, and the
// gfx950 row swaps for m = 16, 32 -- no LDS round trip.
template <class Op>
__device__ __forceinline__ uint32_t wave_reduce64(uint32_t v, Op op) {
    v = op(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xf, 0xf, false));   // [1,0,3,2]
    v = op(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xf, 0xf, false));   // [2,3,0,1]
    v = op(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x141, 0xf, 0xf, false));  // row_half_mirror
    v = op(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x140, 0xf, 0xf, false));  // row_mirror
    const int lane = threadIdx.x & 63;
    // permlane16_swap(v, v) returns (rows 0,0,2,2 ; rows 1,1,3,3) of v
    const auto s16 = __builtin_amdgcn_permlane16_swap((int)v, (int)v, false, false);
    v = op(v, (uint32_t)(((lane >> 4) & 1) ? s16[0] : s16[1]));
    // permlane32_swap(v, v) returns (low, low ; high, high) halves of v
    const auto s32 = __builtin_amdgcn_permlane32_swap((int)v, (int)v, false, false);
    v = op(v, (uint32_t)((lane >> 5) ? s32[0] : s32[1]));
    return v;
}

// Balanced pairwise sum of the 64 values (the lower six levels of
// gdn_tree_reduce_256); FP32 addition is commutative, so the sums equal an
// XOR butterfly's.
__device__ __forceinline__ float wave_tree64(float v) {
    return u2f(wave_reduce64(f2u(v), [](uint32_t a, uint32_t b) { return f2u(u2f(a) + u2f(b)); }));
}

// Balanced pairwise sum of each 32-lane half's values (the lower five levels
// of gdn_tree_reduce_256 over 32 consecutive values), left in every lane of
// the half.
__device__ __forceinline__ float wave_tree32(float v) {
    auto add = [](uint32_t a, uint32_t b) { return f2u(u2f(a) + u2f(b)); };
    uint32_t u = f2u(v);
    u = add(u, (uint32_t)__builtin_amdgcn_mov_dpp((int)u, 0xB1, 0xf, 0xf, false));
    u = add(u, (uint32_t)__builtin_amdgcn_mov_dpp((int)u, 0x4E, 0xf, 0xf, false));
    u = add(u, (uint32_t)__builtin_amdgcn_mov_dpp((int)u, 0x141, 0xf, 0xf, false));
    u = add(u, (uint32_t)__builtin_amdgcn_mov_dpp((int)u, 0x140, 0xf, 0xf, false));
    const int lane = threadIdx.x & 63;
    const auto s16 = __builtin_amdgcn_permlane16_swap((int)u, (int)u, false, false);
    u = add(u, (uint32_t)(((lane >> 4) & 1) ? s16[0] : s16[1]));
    return u2f(u);
}

// Sum over lane quads (lanes 4i..4i+3) in XOR-butterfly pairing, in every
// lane of the quad.
__device__ __forceinline__ float quad_sum(float v) {
    v = v + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xf, 0xf, false));
    return v + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xf, 0xf, false));
}

// Two FP32 values to a BF16 pair (lo in bits 0..15), round to nearest even
// (v_cvt_pk_bf16_f32; equal to the integer rounding for every non-NaN input).
__device__ __forceinline__ uint32_t cvt_pk(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, bf16x2));
}

// beta = sigmoid(b); decay = expf(-expf(a_log) * softplus(a + dt_bias))
// (gdn_island_prep, gdn_model.cpp:2461-2465).
template <class Tab = Exp2Const>
__device__ __forceinline__ void head_scalars(float a, float b, float a_log, float dt_bias,
                                             float &beta, float &decay, const Tab &tab = Tab()) {
    beta = sigmoid_ref(b, tab);
    const float decay_in = a + dt_bias;
    const float decay_val = -exp_ref(a_log, tab) * softplus_ref(decay_in, tab);
    decay = exp_ref(decay_val, tab);
}

// Recurrent-state layouts.  Row-major: head h, key row j, value column i
// at h*65536 + j*256 + i (the .gdnstate order).  Tiled: the 256 x CB tile
// of columns [c0, c0 + CB) is contiguous, rows in order, so a workgroup
// owning one tile reads and writes whole cache lines:
// h*65536 + (c0/CB)*256*CB + j*CB + (i - c0).
template <bool TILED, int CB>
__device__ __forceinline__ size_t state_index(int h, int j, int c0) {
    if constexpr (TILED) return (size_t)h * kHD * kHD + (size_t)(c0 / CB) * kHD * CB + (size_t)j * CB;
    else return (size_t)h * kHD * kHD + (size_t)j * kHD + c0;
}

// A load of one float through a vector memory instruction: the address is
// moved into VGPRs first, so a uniform address does not become a scalar load
// (whose wait, lgkmcnt, would also hold back unrelated scalar loads).
__device__ __forceinline__ float vector_load(const float *p) {
    asm volatile("" : "+v"(p));
    return *(const __attribute__((address_space(1))) float *)p;
}

// Four consecutive floats (16-byte aligned) through one vector memory
// instruction, for the same reason as vector_load.
__device__ __forceinline__ f32x4 vector_load4(const float *p) {
    asm volatile("" : "+v"(p));
    return *(const __attribute__((address_space(1))) f32x4 *)p;
}

// Per-head (beta, decay) for recur_block: read from precomputed pairs, or
// computed from the raw a_h and b_h (head_scalars).  read() issues the loads
// (after the state loads), get() returns the pair; recur_block evaluates it
// on wave 3 while wave 0 runs the column chains.
struct ScalarsFromPairs {
    const float *bd;
    float v[2];
    __device__ __forceinline__ void read(int h) {
        v[0] = vector_load(bd + 2 * h);
        v[1] = vector_load(bd + 2 * h + 1);
    }
    template <class Tab>
    __device__ __forceinline__ void get(float &beta, float &decay, const Tab &) const {
        beta = v[0];
        decay = v[1];
    }
};
struct ScalarsFromAB {
    const float *a, *b, *a_log, *dt_bias;
    float v[4];
    __device__ __forceinline__ void read(int h) {
        v[0] = vector_load(a + h);
        v[1] = vector_load(b + h);
        v[2] = vector_load(a_log + h);
        v[3] = vector_load(dt_bias + h);
    }
    template <class Tab>
    __device__ __forceinline__ void get(float &beta, float &decay, const Tab &tab) const {
        head_scalars(v[0], v[1], v[2], v[3], beta, decay, tab);
    }
};

// Gated delta rule for one head and CB state columns, run by one workgroup
// of 256 threads; thread t holds key row t of the tile (CB columns) in
// registers.  beta/decay come from scal, evaluated while the state loads
// are in flight.
//   q/k L2 norms in gdn_tree_reduce_256 order: with PRE the QKVG kernel
//   has already reduced each 16-row block (the tree's lower four levels;
//   qk_part[h*16 + b], k at offset 128) and the top four levels run here,
//   otherwise four wave butterflies then (w0 + w1) + (w2 + w3);
//   alpha = tree256(qn * kn) (only o needs it, after the chains);
//   every product S[j][i] * kn[j] and S[j][i] * qn[j] is formed in parallel
//   into column-major LDS tiles, then lane i runs the r_i chain and lane
//   CB + i the p_i chain over j = 0..255 in order (only the dependent adds
//   are serial); delta and o; the update S' = decay * S + kn (x) delta is
//   applied to the tile still held in registers.
//   With OSUM (CB = 16: one tile is one 16-value chunk of the output norm)
//   the workgroup also writes sum_i R(o_i)^2 in order, the chunk's sum of
//   squares, to o_sum[h*16 + c0/16].
template <int C, int CB, bool TILED, bool PRE, bool OSUM, bool ST = false, class Scal>
__device__ __forceinline__ void recur_block(const float *__restrict__ qp, const float *__restrict__ kp,
                                            const float *__restrict__ vp, Scal scal,
                                            const float *__restrict__ qk_part, void *__restrict__ state,
                                            float *__restrict__ attn, float *__restrict__ o_sum, const int h,
                                            const int c0, uint64_t *stamps = nullptr, const int wg = 0) {
    static_assert(CB == 16 || CB == 32, "one wave runs both chains of every column; a thread holds one row");
    static_assert(!OSUM || CB == 16, "an output-norm chunk is 16 columns");
    constexpr int EPT = CB;                             // state elements per thread (its row)
    constexpr int LDT = kHD + 4;                        // padded column stride of the product tiles
    __shared__ __attribute__((aligned(16))) float pk_t[CB * LDT];  // S[j][i] * kn[j] at [i][j]
    __shared__ __attribute__((aligned(16))) float pq_t[CB * LDT];  // S[j][i] * qn[j] at [i][j]
    __shared__ float dl[CB];
    __shared__ float red[8], red2[4], bdsh[2];
    __shared__ uint64_t exp2_lds[32];
    const int t = threadIdx.x;
    const int lane = t & 63, w = t >> 6;
    const size_t sidx = state_index<TILED, CB>(h, t, c0);
    Exp2Fill e2;
    phase_stamp<ST>(stamps, wg, 0);

    // With PRE the head's 16 + 16 norm partials are requested first: loads
    // complete in issue order, so behind the state tile their wait would
    // also wait for the tile, and the norms could not run while it arrives.
    // They go through vector loads: as scalar loads (their address is
    // uniform) the wait for the kernel arguments, which the state's address
    // needs, would also wait for them.
    f32x4 qpart[PRE ? 4 : 1], kpart[PRE ? 4 : 1];
    if constexpr (PRE) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            qpart[i] = vector_load4(qk_part + h * 16 + 4 * i);
            kpart[i] = vector_load4(qk_part + 128 + h * 16 + 4 * i);
        }
    }
    const float q = qp[h * kHD + t], k = kp[h * kHD + t];
    const float vi = (t < CB) ? vp[h * kHD + c0 + t] : 0.0f;
    float sv[EPT];  // S[t][c0 + e]
    {
        constexpr int NV = (C == kRef) ? EPT / 8 : EPT / 4;
        u32x4 tr[NV];
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            if constexpr (C == kRef)
                tr[i] = reinterpret_cast<const u32x4 *>(reinterpret_cast<const uint16_t *>(state) + sidx)[i];
            else
                tr[i] = reinterpret_cast<const u32x4 *>(reinterpret_cast<const float *>(state) + sidx)[i];
        }
        scal.read(h);
        e2.load();
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const uint32_t wv[4] = {tr[i].x, tr[i].y, tr[i].z, tr[i].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if constexpr (C == kRef) {
                    sv[8 * i + 2 * e] = u2f(wv[e] << 16);
                    sv[8 * i + 2 * e + 1] = u2f(wv[e] & 0xffff0000u);
                } else {
                    sv[4 * i + e] = u2f(wv[e]);
                }
            }
        }
    }

    float q_sq, k_sq;
    if constexpr (PRE) {
        float qv[16], kv[16];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const f32x4 a = qpart[i], b = kpart[i];
            qv[4 * i] = a.x; qv[4 * i + 1] = a.y; qv[4 * i + 2] = a.z; qv[4 * i + 3] = a.w;
            kv[4 * i] = b.x; kv[4 * i + 1] = b.y; kv[4 * i + 2] = b.z; kv[4 * i + 3] = b.w;
        }
        q_sq = tree16(qv);
        k_sq = tree16(kv);
    } else {
        const float qs = wave_tree64(q * q), ks = wave_tree64(k * k);
        if (lane == 0) {
            red[w] = qs;
            red[4 + w] = ks;
        }
        __syncthreads();
        q_sq = (red[0] + red[1]) + (red[2] + red[3]);
        k_sq = (red[4] + red[5]) + (red[6] + red[7]);
    }
    const float q_inv = 1.0f / __builtin_sqrtf(q_sq + 1e-6f);
    const float k_inv = 1.0f / __builtin_sqrtf(k_sq + 1e-6f);
    const float qj = q * q_inv, kj = k * k_inv;  // row t's normalised q and k
    const float qk = wave_tree64(qj * kj);
    if (lane == 0) red2[w] = qk;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
        pk_t[e * LDT + t] = sv[e] * kj;
        pq_t[e * LDT + t] = sv[e] * qj;
    }
    e2.store(exp2_lds);
    __syncthreads();
    phase_stamp<ST>(stamps, wg, 1);

    // wave 0: the column chains; meanwhile wave 3 evaluates beta and decay
    float acc = 0.0f, pv = 0.0f;
    if (t < 2 * CB) {
        // lane i: r_i = sum_j S[j][i] kn[j]; lane CB + i: p_i (same order)
        const bool is_p = t >= CB;
        const int ci = is_p ? t - CB : t;
        const f32x4 *src = reinterpret_cast<const f32x4 *>((is_p ? pq_t : pk_t) + ci * LDT);
        f32x4 col_v[kHD / 4];  // the whole column, read ahead of the serial adds
#pragma unroll
        for (int j4 = 0; j4 < kHD / 4; ++j4) col_v[j4] = src[j4];
#pragma unroll
        for (int j4 = 0; j4 < kHD / 4; ++j4) {
            acc = acc + col_v[j4].x;
            acc = acc + col_v[j4].y;
            acc = acc + col_v[j4].z;
            acc = acc + col_v[j4].w;
        }
        // lane i takes p_i from lane CB + i
        if constexpr (CB == 16) {
            pv = __int_as_float(__builtin_amdgcn_permlane16_swap(__float_as_int(acc), __float_as_int(acc), false,
                                                                 false)[1]);
        } else {
            pv = __shfl(acc, (lane + CB) & 63);
        }
    } else if (w == 3) {
        float b_, d_;
        scal.get(b_, d_, Exp2Lds{exp2_lds});
        if (lane == 0) {
            bdsh[0] = b_;
            bdsh[1] = d_;
        }
    }
    __syncthreads();
    const float beta = bdsh[0], decay = bdsh[1];

    if (t < 2 * CB) {
        const bool is_p = t >= CB;
        float o = 0.0f;
        if (!is_p) {
            const float alpha = (red2[0] + red2[1]) + (red2[2] + red2[3]);
            const float r = acc;
            const float delta = beta * (vi - decay * r);
            o = R<C>(0.0625f * (decay * pv + alpha * delta));
            dl[t] = delta;
            attn[h * kHD + c0 + t] = o;
        }
        if constexpr (OSUM) {
            // the chunk's sum of squares, lanes 0..15 in order from 0.  The
            // lane reads run in every chain lane (not under t == 0), so each
            // lane's square is computed where it is read.
            const uint32_t sq = f2u(o * o);
            float sum = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) sum += u2f((uint32_t)__builtin_amdgcn_readlane((int)sq, i));
            if (t == 0) o_sum[h * (kHD / 16) + c0 / 16] = sum;
        }
    }
    __syncthreads();
    phase_stamp<ST>(stamps, wg, 2);

    float nv[EPT];
#pragma unroll
    for (int e = 0; e < EPT; ++e) nv[e] = decay * sv[e] + kj * dl[e];
    if constexpr (C == kRef) {
#pragma unroll
        for (int i = 0; i < EPT / 8; ++i) {
            u32x4 v;
            v.x = cvt_pk(nv[8 * i + 0], nv[8 * i + 1]);
            v.y = cvt_pk(nv[8 * i + 2], nv[8 * i + 3]);
            v.z = cvt_pk(nv[8 * i + 4], nv[8 * i + 5]);
            v.w = cvt_pk(nv[8 * i + 6], nv[8 * i + 7]);
            if (!(fabsf(nv[8 * i + 0]) <= 3.402823466e38f) || !(fabsf(nv[8 * i + 1]) <= 3.402823466e38f) ||
                !(fabsf(nv[8 * i + 2]) <= 3.402823466e38f) || !(fabsf(nv[8 * i + 3]) <= 3.402823466e38f) ||
                !(fabsf(nv[8 * i + 4]) <= 3.402823466e38f) || !(fabsf(nv[8 * i + 5]) <= 3.402823466e38f) ||
                !(fabsf(nv[8 * i + 6]) <= 3.402823466e38f) || !(fabsf(nv[8 * i + 7]) <= 3.402823466e38f)) {
                // a NaN or infinity: the integer rounding (canonical NaN)
                uint32_t pk[4];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    pk[e] = (f2u(rne_bf16(nv[8 * i + 2 * e])) >> 16) |
                            (f2u(rne_bf16(nv[8 * i + 2 * e + 1])) & 0xffff0000u);
                v.x = pk[0]; v.y = pk[1]; v.z = pk[2]; v.w = pk[3];
            }
            reinterpret_cast<u32x4 *>(reinterpret_cast<uint16_t *>(state) + sidx)[i] = v;
        }
    } else {
#pragma unroll
        for (int i = 0; i < EPT / 4; ++i) {
            f32x4 v;
            v.x = nv[4 * i + 0]; v.y = nv[4 * i + 1]; v.z = nv[4 * i + 2]; v.w = nv[4 * i + 3];
            reinterpret_cast<f32x4 *>(reinterpret_cast<float *>(state) + sidx)[i] = v;
        }
    }
    if constexpr (ST) {
        __syncthreads();
        phase_stamp<ST>(stamps, wg, 3);
    }
}

}  // namespace gdn

#endif

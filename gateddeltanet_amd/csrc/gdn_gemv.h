// gdn_gemv.h -- the CU-resident GEMV's building blocks shared by the
// per-kernel step (gdn_engine.hip) and the persistent step (gdn_persist.hip)
// of libgdn_amd.so: native BF16 products, the fast-path verdict, the input
// lane words, the bank layout and chains, and the weight stream order.  Not
// part of the ABI.
#ifndef GDN_GEMV_H
#define GDN_GEMV_H

#include <type_traits>

#include "gdn_device.h"

namespace gdn {

constexpr int kCB = 16;    // state columns per recurrence workgroup

// Smallest nonzero and largest |w| of a matrix (after DAZ) and whether any
// is not finite.
struct WInfo {
    float min_abs;
    float max_abs;
    int nonfinite;
};

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

__device__ __forceinline__ void lds_load16u(const uint32_t *src, uint32_t *v) {
    const u32x4 *s4 = reinterpret_cast<const u32x4 *>(src);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const u32x4 t = s4[q];
        v[4 * q + 0] = t.x;
        v[4 * q + 1] = t.y;
        v[4 * q + 2] = t.z;
        v[4 * q + 3] = t.w;
    }
}

// Eight BF16 x BF16 products rounded to BF16, packed in pairs: r[j] holds
// R(w[j].lo * x[2j]) in bits 0..15 and R(w[j].hi * x[2j+1]) in bits 16..31.
// Each product is one v_dot2_f32_bf16 with a zero accumulator: the
// activation word carries its BF16 in the lane of the weight it meets and
// zero in the other lane, so the dot product is the single FP32 product --
// exact for BF16 operands whose product is a normal FP32 number -- and
// v_cvt_pk_bf16_f32 rounds two of them to nearest even.  A VALU read of a
// v_dot2 result needs 3 wait states on gfx950, which the compiler cannot see
// inside inline assembly: the block issues all eight products, one s_nop,
// then the conversions, so every read is at least 4 slots after its write.
__device__ __forceinline__ void dot8_bf16(const uint32_t *w, const uint32_t *x, uint32_t *r) {
    float t0, t1, t2, t3, t4, t5, t6, t7;
    asm("v_dot2_f32_bf16 %4, %12, %16, 0\n\t"
        "v_dot2_f32_bf16 %5, %12, %17, 0\n\t"
        "v_dot2_f32_bf16 %6, %13, %18, 0\n\t"
        "v_dot2_f32_bf16 %7, %13, %19, 0\n\t"
        "v_dot2_f32_bf16 %8, %14, %20, 0\n\t"
        "v_dot2_f32_bf16 %9, %14, %21, 0\n\t"
        "v_dot2_f32_bf16 %10, %15, %22, 0\n\t"
        "v_dot2_f32_bf16 %11, %15, %23, 0\n\t"
        "s_nop 0\n\t"
        "v_cvt_pk_bf16_f32 %0, %4, %5\n\t"
        "v_cvt_pk_bf16_f32 %1, %6, %7\n\t"
        "v_cvt_pk_bf16_f32 %2, %8, %9\n\t"
        "v_cvt_pk_bf16_f32 %3, %10, %11"
        : "=v"(r[0]), "=v"(r[1]), "=v"(r[2]), "=v"(r[3]), "=&v"(t0), "=&v"(t1), "=&v"(t2),
          "=&v"(t3), "=&v"(t4), "=&v"(t5), "=&v"(t6), "=&v"(t7)
        : "v"(w[0]), "v"(w[1]), "v"(w[2]), "v"(w[3]), "v"(x[0]), "v"(x[1]), "v"(x[2]), "v"(x[3]),
          "v"(x[4]), "v"(x[5]), "v"(x[6]), "v"(x[7]));
}

// Swap values between lane pairs (2i, 2i + 1) with a DPP quad permutation.
__device__ __forceinline__ float swap_lane_pair(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xf, 0xf, false));
}

// Running magnitude statistics of BF16 activation pairs, per 16-bit half:
// the largest |x| bits and the smallest (|x| bits - 1), where zero wraps to
// 0xffff and so never wins.
struct PairStats {
    uint32_t mx = 0u, mnm1 = 0xffffffffu;
    __device__ __forceinline__ void add(uint32_t pair) {
        const u16x2 m = __builtin_bit_cast(u16x2, pair & 0x7fff7fffu);
        const u16x2 one = {1, 1};
        mx = __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2, mx), m));
        mnm1 = __builtin_bit_cast(uint32_t,
                                  __builtin_elementwise_min(__builtin_bit_cast(u16x2, mnm1), (u16x2)(m - one)));
    }
};


// ------------------------------------------------------------------ GEMV core
//
// A workgroup owns RB consecutive rows of the device matrix (row-major, so
// the block is one contiguous stream).  Work item f is one 16-column
// half-beat of one row: row f / (K/16), half-beat f % (K/16), at element
// offset 16 f of the block -- consecutive threads read consecutive 32-byte
// (BF16) or 64-byte (FP32) pieces.  Each item's 16 products are reduced
// in-lane with tree16 into LDS; then lanes 0..4RB-1 of wave 0 each run one
// of the reference's four bank chains (lower/upper half x even/odd beat, in
// beat order from +0.0f) and two XOR shuffles form
// (even_lo + even_hi) + (odd_lo + odd_hi).
//
// Every kernel issues its weight loads before any activation-dependent
// work: the activation prologue (residual add, RMSNorm, output norm * gate)
// runs while the weight stream is in flight, and s_barrier does not wait
// on outstanding global loads.
//
// The GEMV input lives in LDS as one 32-bit word per element.  BF16
// contracts: element k's BF16 bits sit in the half of the word that meets
// weight k in the packed weight pair (low half for even k, high half for odd
// k) and the other half is zero -- the operand form of dot2_bf16, and for odd
// k also the FP32 value itself.  FP32 contract: the FP32 value.

template <int K>
struct Hb {
    static constexpr int HB = K / 16;     // half-beats per row
    static constexpr int HBP = HB + 4;    // padded LDS row stride
    static constexpr int NB = K / 32;     // 32-column beats per row
};

__device__ __forceinline__ float lane_word_value(uint32_t w, int k) {
    return (k & 1) ? u2f(w) : u2f(w << 16);
}


// ---------------------------------------------------------------- prologues

enum { PRO_PLAIN = 0, PRO_RESNORM = 1, PRO_EMBED = 2, PRO_ONORM = 3 };

struct BlockSync {
    __device__ __forceinline__ void operator()() { __syncthreads(); }
};

constexpr int kSpinMax = 1 << 24;

__device__ __forceinline__ void wait_count(int *ctr, int target, int *err) {
    int spins = 0;
    while (__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < target &&
           ++spins < kSpinMax)
        __builtin_amdgcn_s_sleep(1);
    if (spins >= kSpinMax && err != nullptr && (threadIdx.x & 63) == 0)
        __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

struct Wave4Sync {
    int *ctr;
    int *err;
    int phase = 0;
    __device__ __forceinline__ void operator()() {
        ++phase;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        if ((threadIdx.x & 63) == 0)
            __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        wait_count(ctr, 4 * phase, err);
    }
};

// Fast-path verdict (BF16 contracts): every input finite and normal or
// zero, every weight finite, and every product |x| |w| inside
// [2^-123, 2^126) -- so no product reaches the flush threshold or overflows
// and dot2_bf16 + v_cvt_pk_bf16_f32 equal the native product.
// The input-owning waves 0..3 publish their statistics, then any thread
// decides from the published values.
__device__ __forceinline__ void publish_stats(PairStats st, uint32_t *red) {
    uint32_t mx = max(st.mx & 0xffffu, st.mx >> 16);
    uint32_t mn = min(st.mnm1 & 0xffffu, st.mnm1 >> 16);
    mx = wave_reduce64(mx, [](uint32_t a, uint32_t b) { return max(a, b); });
    mn = wave_reduce64(mn, [](uint32_t a, uint32_t b) { return min(a, b); });
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    if (lane == 0 && w < 4) {
        red[w] = mx;
        red[4 + w] = mn;
    }
}

__device__ __forceinline__ bool decide_fast(const uint32_t *red, WInfo wi) {
    const uint32_t mx = max(max(red[0], red[1]), max(red[2], red[3]));
    const uint32_t mn = min(min(red[4], red[5]), min(red[6], red[7]));
    if (mx >= 0x7f80u || wi.nonfinite) return false;  // an input NaN/infinity or a weight
    if (mn == 0xffffu) return true;                     // every input is zero
    const uint32_t mn_mag = mn + 1u;
    if (mn_mag < 0x0080u) return false;                 // a subnormal input
    const double lo = (double)u2f(mn_mag << 16) * (double)wi.min_abs;
    const double hi = (double)u2f(mx << 16) * (double)wi.max_abs;
    return lo >= 0x1p-123 && hi < 0x1p126;
}

// Serial sum of the 128 chunk sums in scratch by wave 0 (the other waves
// wait at the barrier instead of spending issue slots on the same chain);
// every thread returns the total.  Two barriers.
template <class Sync>
__device__ __forceinline__ float chunk_total(const float *scratch, float *bcast, Sync &sync) {
    sync();
    const int t = threadIdx.x;
    if (t < 64) {
        const f32x4 *s4 = reinterpret_cast<const f32x4 *>(scratch);
        float sum = 0.0f;
#pragma unroll 8
        for (int i = 0; i < kH / 64; ++i) {
            const f32x4 c = s4[i];
            sum += c.x;
            sum += c.y;
            sum += c.z;
            sum += c.w;
        }
        if (t == 0) bcast[0] = sum;
    }
    sync();
    return bcast[0];
}

// Sum of squares of 16-value chunks in order, when thread 2c holds the first
// 8 values of chunk c and thread 2c + 1 the last 8: the even lane's running
// sum moves to the odd lane, which finishes the chunk.  Odd lanes return the
// chunk sum.
__device__ __forceinline__ float chunk_sumsq8(const float *r) {
    float sq[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) sq[e] = r[e] * r[e];
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) s += sq[e];
    float c = swap_lane_pair(s);
#pragma unroll
    for (int e = 0; e < 8; ++e) c += sq[e];
    return c;
}

// Store 8 (BF16 pairs ->) lane words for elements [8t, 8t + 8).
__device__ __forceinline__ void store_pairs8(uint32_t *xs, const uint32_t *pairs, PairStats &st) {
    u32x4 lo, hi;
    uint32_t lw[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        st.add(pairs[j]);
        lw[2 * j] = pairs[j] & 0xffffu;
        lw[2 * j + 1] = pairs[j] & 0xffff0000u;
    }
    lo.x = lw[0]; lo.y = lw[1]; lo.z = lw[2]; lo.w = lw[3];
    hi.x = lw[4]; hi.y = lw[5]; hi.z = lw[6]; hi.w = lw[7];
    u32x4 *d = reinterpret_cast<u32x4 *>(xs + 8 * threadIdx.x);
    d[0] = lo;
    d[1] = hi;
}

__device__ __forceinline__ void unpack8(const f32x4 *v, float *o) {
    o[0] = v[0].x; o[1] = v[0].y; o[2] = v[0].z; o[3] = v[0].w;
    o[4] = v[1].x; o[5] = v[1].y; o[6] = v[1].z; o[7] = v[1].w;
}

// ---------------------------------------------------------------- epilogues

enum { EPI_RAW = 0, EPI_STORE = 1, EPI_QKVG = 2, EPI_SWIGLU = 3, EPI_LM = 4 };

// ------------------------------------------------ CU-resident GEMV
//
// One 1024-thread workgroup per CU (it claims all 512 VGPRs of every SIMD,
// so no two share one) owns ROWS consecutive rows of the matrix, a
// contiguous slice of the weight stream, as 16-element items held in
// registers (WStream).  Waves 0..3 read the activations and build the GEMV
// input (residual add, norms) once per CU while the weights stream in.  The
// vector memory path of a CU serves requests in order, so the activation
// reads are issued before the weight loads: in the input-first kernels a
// barrier orders them ahead of every weight load and only waves 4..15 carry
// items; in gate/up and down all 16 waves stream.
constexpr int kTB = 1024;  // threads per CU-resident workgroup
// Rows per CU-resident workgroup (grids of 256 workgroups).
constexpr int kCuQkvg = 32;   // 8192 / 256
constexpr int kCuO = 8;       // 2048 / 256
constexpr int kCuGu = 44;     // 22 gate + 22 up rows: 11264 / 256
constexpr int kCuDown = 8;    // 2048 / 256
constexpr int kCuLm = 125;    // 32000 / 256
constexpr int kCuLmSmall = 8; // vocabularies that 125 does not divide
// Items in flight per thread (16 = every item issued up front).  QKVG and
// gate/up hold 6 items per thread, down 3, the LM head 21.  With the
// stream-order layout, priming 3 of QKVG's, 2 of gate/up's, all 3 of down's
// and 3 of the LM head's measured 3 % faster per token than 4 / 3 / 2 / 2
// (the best mix of the earlier layout); gate/up at 1, QKVG at 2 or 6 were
// slower.
constexpr int kDepthAll = 16;
constexpr int kDepthQkvg = 3;
constexpr int kDepthGu = 2;
constexpr int kDepthDown = 3;
constexpr int kDepthLm = 3;
// Per contract: an FP32 item is 64 bytes (16 VGPRs), so the FP32 control
// arm keeps fewer in flight within the same 128-VGPR budget.
template <int C>
struct Depth {
    static constexpr bool F = C == kFp32;
    static constexpr int qkvg = F ? 3 : kDepthQkvg;
    static constexpr int o = F ? 2 : kDepthAll;
    static constexpr int gu = F ? 3 : kDepthGu;
    static constexpr int down = F ? 2 : kDepthDown;
    static constexpr int lm = F ? 2 : kDepthLm;
    static constexpr int lm_small = F ? 2 : kDepthAll;
};

// Partial sums of the CU-resident GEMV, bank-contiguous: row r, bank
// (beat parity, half) = 2 * (beat & 1) + half, position beat / 2.  A bank
// segment is padded to 4 (mod 32) words so the four chain lanes of a row
// read distinct LDS banks.
template <int K>
struct BankLayout {
    static constexpr int NB2 = Hb<K>::NB / 2;                       // beats per bank chain
    static constexpr int BSTR = ((NB2 + 3) / 4) * 4 + ((((NB2 + 3) / 4) * 4) % 32 == 4 ? 0 : 4);
    static constexpr int RSTR = 4 * BSTR;
    __device__ static constexpr int index(int row, int hb) {
        return row * RSTR + (2 * ((hb >> 1) & 1) + (hb & 1)) * BSTR + (hb >> 2);
    }
};

// Input-first GEMVs (QKVG, o_proj, LM head): waves 0..3 build the input and
// own no weight items, so kTB - kT threads stream; the others stream on all
// kTB threads.
constexpr bool act_first(int pro, int epi) { return epi == EPI_QKVG || pro == PRO_ONORM || epi == EPI_LM; }
constexpr int stream_threads(int pro, int epi) { return act_first(pro, epi) ? kTB - kT : kTB; }

// Device order of a workgroup's weight slice.  Item f (16 elements: row
// f / (K/16), half-beat f % (K/16)) is held by stream thread u = f % NT as its
// item I = f / NT and arrives in WPI 16-byte pieces (2 for BF16, 4 for FP32).
// Piece q of every item of group I of the NT threads is stored contiguously,
// so each load instruction of a wave reads 1 KB of consecutive bytes: piece
// (f, q) sits at 16-byte position NT WPI I + q span + u, span = NT (or the
// item count of the last group when NT does not divide the items).
__host__ __device__ constexpr size_t stream_piece(int f, int q, int items, int nt, int wpi) {
    const int I = f / nt, u = f - I * nt;
    const int full = items / nt;  // complete groups
    const int span = I < full ? nt : items - full * nt;
    return (size_t)nt * wpi * I + (size_t)q * span + u;
}

template <int K, int CR>
__device__ __forceinline__ float chain_rows(const float *part) {
    using BL = BankLayout<K>;
    constexpr int NV = (BL::NB2 + 3) / 4;
    const int L = threadIdx.x;
    float acc = 0.0f;
    if (L < CR * 4) {
        const f32x4 *seg = reinterpret_cast<const f32x4 *>(part + (L >> 2) * BL::RSTR + (L & 3) * BL::BSTR);
        f32x4 v[NV];
#pragma unroll
        for (int i = 0; i < NV; ++i) v[i] = seg[i];
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            if (4 * i + 0 < BL::NB2) acc = acc + v[i].x;
            if (4 * i + 1 < BL::NB2) acc = acc + v[i].y;
            if (4 * i + 2 < BL::NB2) acc = acc + v[i].z;
            if (4 * i + 3 < BL::NB2) acc = acc + v[i].w;
        }
    }
    return quad_sum(acc);  // (lo + hi) per parity, then the two parities
}

template <int N>
using IC = std::integral_constant<int, N>;

}  // namespace gdn

#endif

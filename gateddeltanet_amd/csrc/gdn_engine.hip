// gdn_engine.hip -- device half of libgdn_amd.so: the CDNA4 (gfx950) kernels
// of one batch-1 GatedDeltaNet decode step, the device layout of weights and
// state, the captured per-token hipGraph, and the run-state entry points of
// include/gdn_amd.h.
//
// One decode step (token id -> argmax token id) is one captured hipGraph of
// 122 launches.  Per layer l (every contract; the FP32 control arm streams
// FP32 weights through the same kernels):
//   QKVG    k_gemv_cu: residual add + attention RMSNorm prologue (the
//           embedding import in layer 0), BF16 GEMV [4H x H] (q,k,v,g),
//           per-channel causal conv/SiLU with the conv-tail shift, gate and
//           sigmoid(gate); workgroup h < 8 also runs head h's tiny a/b rows
//           and beta/decay               gdn_model.cpp:3716-3740, :3785-3797,
//                                        :1394-1474, :1501-1667, :2461-2465
//   recur   k_recur per (head, 16 columns): q/k L2 norms, the Sk / Sq column
//           chains, delta, o and the rank-1 state update  :2376-2933, :3226-3349
//   o_proj  k_gemv_cu: per-head output RMSNorm * gate prologue, GEMV  :3803-3814
//   GU      k_gemv_cu: residual add + MLP RMSNorm prologue, gate/up GEMV
//           (22 + 22 rows per workgroup), SwiGLU  :3815-3826, :4751-4767, :3379-3450
//   down    k_gemv_cu: GEMV [H x I]      :3827-3842
// then the LM head (final norm prologue, FP32 logits, per-workgroup argmax)
// and k_argmax (:3857-3890, :4778-4931).
//
// Arithmetic follows the reference's all-BF16 contract bit for bit (products
// rounded to BF16 with DAZ/FTZ, tree16 + four-bank reduction, every operator
// output rounded to BF16); expf/log1pf are glibc's methods restated
// (gdn_libm.h), so they match the reference's C library bit for bit too.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <type_traits>
#include <vector>

#include "gdn_amd.h"
#include "gdn_device.h"
#include "gdn_gemv.h"
#include "gdn_internal.h"
#include "gdn_persist.h"

namespace gdn {


// Where a GEMV's input vector comes from.
//   PRO_PLAIN    x = a[0..K)
//   PRO_RESNORM  r = b ? R(a + b) : a (the residual add, gdn_bf16_add_half),
//                x = RMSNorm(r) * w (gdn_rmsnorm_rows_bf16 order)
//   PRO_EMBED    r = R(row tok[0] of emb), x = RMSNorm(r) * w
//   PRO_ONORM    x = per-head RMSNorm(a) * w * b * c with b the gate and c
//                its sigmoid (gdn_output_norm_and_gate)
// Block 0 also stores r in res_out and, for PRO_RESNORM, x in aux_out (the
// final hidden vector before the LM head); for PRO_EMBED aux_out receives
// the FP32 embedding row (workspace X).
struct XSrc {
    const float *a, *b, *c;
    const void *emb;
    const int *tok;
    const float *w;
    float *res_out;
    float *aux_out;
    const float *osum; // PRO_ONORM (BF16): the output norm's 16-value chunk sums [8 heads][16]
    int *err;          // host-mapped error word: set when a bounded wait runs out
    uint32_t *xdump;   // when set, workgroup 0 stores its GEMV input (K lane words) and fast-path verdict
    uint64_t *stamps;  // the stamped kernels (ST): each workgroup's phase stamps
    int vocab;
    float eps;
};

// Workgroup barriers for the input prologue.  BlockSync is s_barrier.
// Wave4Sync joins waves 0..3 only -- the waves that own the input elements
// in a CU-resident workgroup -- so they never wait for the other waves,
// which may sit for microseconds issuing their weight loads (a SIMD holds
// only about one wave's worth of outstanding loads).  Each wave's lane 0
// adds one to an LDS arrival counter; the waves spin (s_sleep) until it
// reaches 4 x phase.  The spin is bounded so no wave can hang; the bound
// (about a second) is never reached while the four waves run; if it were,
// the wave sets the error word, which the host turns into a failed step.

// The GEMV input for one workgroup.  load() issues the activation reads (the
// kernel issues the weight stream right after), finish() builds the input in
// LDS and returns the fast-path verdict (after a barrier).
//   BF16 contracts: thread t owns elements [PER t, PER t + PER).  Roundings
//   use v_cvt_pk_bf16_f32; where a NaN may reach a stored BF16 value (the
//   residual and final-hidden outputs) the integer rounding with its
//   canonical NaN is used instead.
//   FP32 contract: thread t owns elements t + 256 m.
template <int C, int K, int PRO>
struct Prologue {
    static constexpr int PER = K / kT;
    static constexpr bool BF = C != kFp32;
    static_assert(!BF || PRO == PRO_PLAIN || PER == 8, "normalised inputs: 8 per thread");
    f32x4 a4[2], b4[2], c4[2], w4[2];
    f32x4 os4[4];  // PRO_ONORM (BF16): the thread's head's 16 output-norm chunk sums
    f32x2 p2[PER / 2];
    u32x4 e4;
    float va[PER], vb[PER], vc[PER], vw[PER];
    int tok = 0;

    __device__ __forceinline__ void load(const XSrc &src) {
        const int t = threadIdx.x;
        if constexpr (PRO == PRO_EMBED) {
            tok = src.tok[0];
            if (tok < 0 || tok >= src.vocab) tok = 0;  // the host rejects these first
        }
        if constexpr (BF) {
            if constexpr (PRO == PRO_PLAIN) {
                const f32x2 *a = reinterpret_cast<const f32x2 *>(src.a) + (size_t)t * (PER / 2);
#pragma unroll
                for (int j = 0; j < PER / 2; ++j) p2[j] = a[j];
            } else if constexpr (PRO == PRO_RESNORM) {
                const f32x4 *a = reinterpret_cast<const f32x4 *>(src.a) + 2 * t;
                const f32x4 *w = reinterpret_cast<const f32x4 *>(src.w) + 2 * t;
                a4[0] = a[0];
                a4[1] = a[1];
                if (src.b) {
                    const f32x4 *b = reinterpret_cast<const f32x4 *>(src.b) + 2 * t;
                    b4[0] = b[0];
                    b4[1] = b[1];
                }
                w4[0] = w[0];
                w4[1] = w[1];
            } else if constexpr (PRO == PRO_EMBED) {
                e4 = *reinterpret_cast<const u32x4 *>(reinterpret_cast<const uint16_t *>(src.emb) +
                                                      (size_t)tok * kH + 8 * t);
                const f32x4 *w = reinterpret_cast<const f32x4 *>(src.w) + 2 * t;
                w4[0] = w[0];
                w4[1] = w[1];
            } else {
                const f32x4 *a = reinterpret_cast<const f32x4 *>(src.a) + 2 * t;
                const f32x4 *g = reinterpret_cast<const f32x4 *>(src.b) + 2 * t;
                const f32x4 *s = reinterpret_cast<const f32x4 *>(src.c) + 2 * t;
                const f32x4 *w = reinterpret_cast<const f32x4 *>(src.w) + 2 * (t & 31);
                // elements 8t.. belong to head t / 32; its 16 chunk sums are
                // read here, ahead of the weight stream
                const f32x4 *cs4 = reinterpret_cast<const f32x4 *>(src.osum + (t >> 5) * (kHD / 16));
                a4[0] = a[0];
                a4[1] = a[1];
                b4[0] = g[0];
                b4[1] = g[1];
                c4[0] = s[0];
                c4[1] = s[1];
                w4[0] = w[0];
                w4[1] = w[1];
#pragma unroll
                for (int i = 0; i < 4; ++i) os4[i] = cs4[i];
            }
        } else {
            if constexpr (PRO == PRO_PLAIN) {
#pragma unroll
                for (int m = 0; m < PER; ++m) va[m] = src.a[t + kT * m];
            } else if constexpr (PRO == PRO_RESNORM) {
#pragma unroll
                for (int m = 0; m < PER; ++m) {
                    va[m] = src.a[t + kT * m];
                    vb[m] = src.b ? src.b[t + kT * m] : 0.0f;
                    vw[m] = src.w[t + kT * m];
                }
            } else if constexpr (PRO == PRO_EMBED) {
#pragma unroll
                for (int m = 0; m < PER; ++m) {
                    va[m] = reinterpret_cast<const float *>(src.emb)[(size_t)tok * kH + t + kT * m];
                    vw[m] = src.w[t + kT * m];
                }
            } else {
#pragma unroll
                for (int m = 0; m < PER; ++m) {
                    va[m] = src.a[t + kT * m];
                    vb[m] = src.b[t + kT * m];
                    vc[m] = src.c[t + kT * m];
                }
                vw[0] = src.w[t];
            }
        }
    }

    // barriers finish_bf16 passes through
    static constexpr int kSyncs = (PRO == PRO_PLAIN || PRO == PRO_ONORM) ? 1 : 3;

    // BF16 contracts: called by threads 0..255 (the element owners); every
    // barrier is sync(), kSyncs of them.
    template <class Sync>
    __device__ __forceinline__ bool finish_bf16(const XSrc &src, WInfo wi, uint32_t *xs,
                                                float *scratch, float *bcast, uint32_t *red,
                                                Sync &sync) {
        const int t = threadIdx.x;
        const bool act = t < kT;
        PairStats st;
        if constexpr (PRO == PRO_PLAIN) {
            // the BF16 of each element is its top half (the reference's
            // activation conversion), placed in its lane
            if (act) {
#pragma unroll
                for (int j = 0; j < PER / 2; ++j) {
                    const uint32_t b0 = f2u(p2[j].x), b1 = f2u(p2[j].y);
                    const uint32_t pair = (b1 & 0xffff0000u) | (b0 >> 16);
                    st.add(pair);
                    u32x2 lw;
                    lw.x = pair & 0xffffu;
                    lw.y = pair & 0xffff0000u;
                    reinterpret_cast<u32x2 *>(xs + PER * t)[j] = lw;
                }
            }
        } else if constexpr (PRO == PRO_RESNORM || PRO == PRO_EMBED) {
            float r[8], w[8];
            if (act) {
                float a[8], b[8];
                unpack8(w4, w);
                if constexpr (PRO == PRO_EMBED) {
                    const uint32_t e[4] = {e4.x, e4.y, e4.z, e4.w};
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        r[2 * j] = u2f(e[j] << 16);
                        r[2 * j + 1] = u2f(e[j] & 0xffff0000u);
                    }
                } else {
                    unpack8(a4, a);
                    if (src.b) {
                        unpack8(b4, b);
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const uint32_t rp = cvt_pk(a[2 * j] + b[2 * j], a[2 * j + 1] + b[2 * j + 1]);
                            r[2 * j] = u2f(rp << 16);
                            r[2 * j + 1] = u2f(rp & 0xffff0000u);
                        }
                    } else {
#pragma unroll
                        for (int e = 0; e < 8; ++e) r[e] = a[e];
                    }
                }
                const float cs = chunk_sumsq8(r);
                if (t & 1) scratch[t >> 1] = cs;
            }
            const float sum = chunk_total(scratch, bcast, sync);
            if (act) {
                const bool finite = sum <= 3.402823466e38f;
                if (blockIdx.x == 0) {
                    // stored BF16 values: exact rounding, canonical NaN (a NaN
                    // or infinity is rare: the inputs are read again)
                    float rs[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) rs[e] = r[e];
                    if (!finite) {
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            if constexpr (PRO == PRO_EMBED) rs[e] = rne_bf16(r[e]);
                            else if (src.b) rs[e] = rne_bf16(src.a[8 * t + e] + src.b[8 * t + e]);
                        }
                    }
                    if (src.res_out) {
                        f32x4 *d = reinterpret_cast<f32x4 *>(src.res_out) + 2 * t;
                        d[0] = (f32x4){rs[0], rs[1], rs[2], rs[3]};
                        d[1] = (f32x4){rs[4], rs[5], rs[6], rs[7]};
                    }
                    if constexpr (PRO == PRO_EMBED) {
                        if (src.aux_out) {  // the FP32 embedding row as read
                            f32x4 *d = reinterpret_cast<f32x4 *>(src.aux_out) + 2 * t;
                            d[0] = (f32x4){r[0], r[1], r[2], r[3]};
                            d[1] = (f32x4){r[4], r[5], r[6], r[7]};
                        }
                    }
                }
                const float scale = 1.0f / __builtin_sqrtf(sum / (float)kH + src.eps);
                float xv[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) xv[e] = r[e] * scale * w[e];
                uint32_t pairs[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) pairs[j] = cvt_pk(xv[2 * j], xv[2 * j + 1]);
                store_pairs8(xs, pairs, st);
                if constexpr (PRO == PRO_RESNORM) {
                    if (blockIdx.x == 0 && src.aux_out) {
                        // x from the rounded residual (a NaN there makes every
                        // x NaN; only its bits need the canonical form)
                        f32x4 *d = reinterpret_cast<f32x4 *>(src.aux_out) + 2 * t;
                        float xo[8];
#pragma unroll
                        for (int e = 0; e < 8; ++e) xo[e] = rne_bf16(xv[e]);
                        d[0] = (f32x4){xo[0], xo[1], xo[2], xo[3]};
                        d[1] = (f32x4){xo[4], xo[5], xo[6], xo[7]};
                    }
                }
            }
        } else {
            // per-head sums of squares: the recurrence wrote each 16-value
            // chunk's sum (one chunk per recurrence workgroup); every thread
            // adds its head's 16 chunk sums in order itself
            if (act) {
                float a[8], g[8], sg[8], w[8];
                unpack8(a4, a);
                unpack8(b4, g);
                unpack8(c4, sg);
                unpack8(w4, w);
                float sum = 0.0f;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const f32x4 c = os4[i];
                    sum += c.x;
                    sum += c.y;
                    sum += c.z;
                    sum += c.w;
                }
                const float sc = 1.0f / __builtin_sqrtf(sum / (float)kHD + src.eps);
                uint32_t pairs[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float x0 = a[2 * j] * sc * w[2 * j] * g[2 * j] * sg[2 * j];
                    const float x1 = a[2 * j + 1] * sc * w[2 * j + 1] * g[2 * j + 1] * sg[2 * j + 1];
                    pairs[j] = cvt_pk(x0, x1);
                }
                store_pairs8(xs, pairs, st);
            }
        }
        publish_stats(st, red);
        sync();
        return decide_fast(red, wi);
    }

    // FP32 contract: the same operators with every rounding point the
    // identity; products are plain FP32 (no fast path needed).  Called by
    // threads 0..255; every barrier is sync(), kSyncsFp32 of them.
    static constexpr int kSyncsFp32 = (PRO == PRO_PLAIN) ? 1 : 4;

    template <class Sync>
    __device__ __forceinline__ bool finish_fp32(const XSrc &src, float *xs, float *scratch,
                                                float *bcast, Sync &sync) {
        const int t = threadIdx.x;
        if constexpr (PRO == PRO_PLAIN) {
#pragma unroll
            for (int m = 0; m < PER; ++m) xs[t + kT * m] = va[m];
        } else if constexpr (PRO == PRO_RESNORM || PRO == PRO_EMBED) {
            const bool blk0 = blockIdx.x == 0;
#pragma unroll
            for (int m = 0; m < PER; ++m) {
                float r;
                if constexpr (PRO == PRO_EMBED) {
                    r = va[m];
                    if (blk0 && src.aux_out) src.aux_out[t + kT * m] = va[m];
                } else {
                    r = src.b ? va[m] + vb[m] : va[m];
                }
                va[m] = r;
                xs[t + kT * m] = r;
                if (blk0 && src.res_out) src.res_out[t + kT * m] = r;
            }
            sync();
            if (t < kH / 16) {
                float s = 0.0f;
#pragma unroll
                for (int kk = 0; kk < 16; ++kk) {
                    const float v = xs[16 * t + kk];
                    s += v * v;
                }
                scratch[t] = s;
            }
            const float sum = chunk_total(scratch, bcast, sync);
            const float scale = 1.0f / __builtin_sqrtf(sum / (float)kH + src.eps);
#pragma unroll
            for (int m = 0; m < PER; ++m) {
                const float xn = va[m] * scale * vw[m];
                xs[t + kT * m] = xn;
                if constexpr (PRO == PRO_RESNORM) {
                    if (blk0 && src.aux_out) src.aux_out[t + kT * m] = xn;
                }
            }
        } else {
#pragma unroll
            for (int m = 0; m < PER; ++m) xs[t + kT * m] = va[m];
            sync();
            if (t < kNH * (kHD / 16)) {
                float s = 0.0f;
#pragma unroll
                for (int kk = 0; kk < 16; ++kk) {
                    const float v = xs[16 * t + kk];
                    s += v * v;
                }
                scratch[t] = s;
            }
            sync();
            if (t < kNH) {
                float sum = 0.0f;
#pragma unroll
                for (int ch = 0; ch < kHD / 16; ++ch) sum += scratch[t * (kHD / 16) + ch];
                bcast[t] = 1.0f / __builtin_sqrtf(sum / (float)kHD + src.eps);
            }
            sync();
#pragma unroll
            for (int m = 0; m < PER; ++m) {  // element t + 256 m belongs to head m
                const float normalized = va[m] * bcast[m] * vw[0];
                xs[t + kT * m] = normalized * vb[m] * vc[m];
            }
        }
        sync();
        return false;
    }
};


struct Epi {
    float *y;          // RAW/STORE/SWIGLU/LM: results; QKVG: conv outputs q,k,v
    float *y2;         // QKVG: gate
    float *y3;         // QKVG: sigmoid(gate)
    const float *aux;  // QKVG: the layer's small weights
    const uint16_t *ab16;  // QKVG (CU-resident): the layer's a/b rows [16][kH] as BF16 bits
    float *tails;      // QKVG: the layer's conv tails (3 stripes)
    float *ab;         // QKVG: a[8], b[8] (rounded)
    float *qk_part;    // QKVG: q and k sums of squares per 16-row block, [2][8 heads][16]
    float *part_val;   // LM: per-block argmax
    int *part_idx;
};


// A workgroup's weight rows as a stream of 16-element items (stream_piece
// order); stream thread u = threadIdx.x - T0 takes items u + (kTB - T0) i
// (T0 = 256 when waves 0..3 build the input and own no items).  prime()
// issues the loads of the first DEPTH items; run() walks the items in order,
// issuing item i + DEPTH before multiplying item i, so a wave never has more
// than DEPTH items in flight (a SIMD holds only about one wave's worth of
// outstanding loads; a wave that asks for more stalls at issue and cannot
// multiply the items it already has).
template <int K, int ROWS, int C, int D, int T0, bool NTL = true>
struct WStream {
    static constexpr int NT = kTB - T0;  // stream threads
    static constexpr int HB = Hb<K>::HB;
    static constexpr int ITEMS = ROWS * HB;
    static constexpr int NIT = (ITEMS + NT - 1) / NT;
    static constexpr int DEPTH = D < NIT ? D : NIT;
    static constexpr bool kFull = (ITEMS % NT) == 0;
    static constexpr bool kSameHb = (NT % HB) == 0;
    static constexpr int WPI = (C == kFp32) ? 4 : 2;  // 16-byte loads per item
    const u32x4 *wb;
    u32x4 v[NIT][WPI];

    template <int I>
    __device__ __forceinline__ void load() {
        const int u = (int)threadIdx.x - T0;
        if (kFull || u + NT * I < ITEMS) {
            constexpr int span = (kFull || I < NIT - 1) ? NT : ITEMS - NT * (NIT - 1);
#pragma unroll
            for (int q = 0; q < WPI; ++q) {
                const u32x4 *p = wb + (size_t)NT * WPI * I + q * span + u;
                if constexpr (NTL) v[I][q] = __builtin_nontemporal_load(p);
                else v[I][q] = *p;
            }
        }
    }

    template <int I>
    __device__ __forceinline__ void prime_from() {
        if constexpr (I < DEPTH) {
            load<I>();
            prime_from<I + 1>();
        }
    }

    __device__ __forceinline__ void prime(const void *__restrict__ slice) {
        wb = reinterpret_cast<const u32x4 *>(slice);
        prime_from<0>();
    }

    // Item I (compile-time, so the item registers stay registers), then the
    // rest.
    template <bool FAST, int I>
    __device__ __forceinline__ void run_from(const uint32_t *xs, float *part, uint32_t *xv) {
        if constexpr (I < NIT) {
            if constexpr (I + DEPTH < NIT) load<I + DEPTH>();
            const int f = (int)threadIdx.x - T0 + NT * I;
            if (kFull || f < ITEMS) {
                const int row = f / HB, hb = f - row * HB;
                if constexpr (!kSameHb) lds_load16u(xs + hb * 16, xv);
                float p[16];
                if constexpr (C == kFp32) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        p[4 * q + 0] = u2f(v[I][q].x) * u2f(xv[4 * q + 0]);
                        p[4 * q + 1] = u2f(v[I][q].y) * u2f(xv[4 * q + 1]);
                        p[4 * q + 2] = u2f(v[I][q].z) * u2f(xv[4 * q + 2]);
                        p[4 * q + 3] = u2f(v[I][q].w) * u2f(xv[4 * q + 3]);
                    }
                } else if constexpr (FAST) {
                    const uint32_t w8[8] = {v[I][0].x, v[I][0].y, v[I][0].z, v[I][0].w,
                                            v[I][1].x, v[I][1].y, v[I][1].z, v[I][1].w};
                    uint32_t rbits[8];
                    dot8_bf16(w8, xv, rbits);
                    dot8_bf16(w8 + 4, xv + 8, rbits + 4);
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        p[2 * e] = u2f(rbits[e] << 16);
                        p[2 * e + 1] = u2f(rbits[e] & 0xffff0000u);
                    }
                } else {
                    const uint32_t w8[8] = {v[I][0].x, v[I][0].y, v[I][0].z, v[I][0].w,
                                            v[I][1].x, v[I][1].y, v[I][1].z, v[I][1].w};
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        p[2 * e] = native_exact(w8[e] & 0xffffu, u2f(xv[2 * e] << 16));
                        p[2 * e + 1] = native_exact(w8[e] >> 16, u2f(xv[2 * e + 1]));
                    }
                }
                part[BankLayout<K>::index(row, hb)] = tree16(p);
            }
            // keep the scheduler from hoisting later loads above this item
            // (their registers would all be live at once)
            if constexpr (DEPTH < NIT) __builtin_amdgcn_sched_barrier(0);
            run_from<FAST, I + 1>(xs, part, xv);
        }
    }

    template <bool FAST>
    __device__ __forceinline__ void run(const uint32_t *xs, float *part) {
        uint32_t xv[16];
        if constexpr (kSameHb) lds_load16u(xs + ((threadIdx.x - T0) % HB) * 16, xv);
        run_from<FAST, 0>(xs, part, xv);
    }
};

// Bank chains of CR rows: thread L < 4 CR runs chain L & 3 of row L >> 2
// (the waves that hold those threads call this); lane 4r ends with row r.
// The chain's whole bank segment is read before its serial adds.
// ROWS rows per workgroup (grid = M / ROWS), at most D items in flight per
// thread.
//   EPI_QKVG    rows are q|k|v|g; workgroups 0..15 also run one row of the
//               tiny a|b projection
//   EPI_SWIGLU  a workgroup's rows are ROWS/2 gate rows then the matching
//               ROWS/2 up rows
//   EPI_LM      FP32 logits and the workgroup's argmax
// NTS: stream threads (0: stream_threads(PRO, EPI)); the persistent step's
// weight layout is streamed by 512 (waves 8..15).  ST: the instrumented copy
// (phase stamps at start, input ready, products done and end).
template <int C, int K, int ROWS, int D, int PRO, int EPI, int NTS = 0, bool ST = false>
__global__ __launch_bounds__(kTB, 1) void k_gemv_cu(const void *__restrict__ W, WInfo wi, XSrc src,
                                                   Epi ep) {
    constexpr int CR = ROWS;
    constexpr int CHW = (4 * CR + 63) / 64;  // waves that run bank chains
    static_assert(CHW <= 16, "one chain lane per bank");
    static_assert(K % kT == 0 && (PRO == PRO_PLAIN || K == kH), "input shape");
    static_assert(EPI != EPI_QKVG || (K == kH && CHW <= 3), "a/b rows: hidden input; wave 3 runs no bank chain");
    __shared__ __attribute__((aligned(16))) uint32_t xs[K];
    __shared__ __attribute__((aligned(16))) float part[CR * BankLayout<K>::RSTR];
    __shared__ __attribute__((aligned(16))) float scratch[kH / 16];
    __shared__ float bcast[kNH];
    __shared__ uint32_t red[8];
    __shared__ float ybuf[ROWS];
    __shared__ float abpart[Hb<kH>::HB];
    // expf's table for the epilogue's SiLU / sigmoid (QKVG, gate/up)
    constexpr bool kExpTab = EPI == EPI_QKVG || EPI == EPI_SWIGLU;
    __shared__ uint64_t exp2_lds[kExpTab ? 32 : 1];
    // claim the whole register file (128 VGPRs x 16 waves): one workgroup per CU
    asm volatile("" ::: "v127");
    const int t = threadIdx.x, wave = t >> 6;
    phase_stamp<ST>(src.stamps, blockIdx.x, 0);
    constexpr bool BF = C != kFp32;
    const int row0 = blockIdx.x * ROWS;
    const char *wblk = static_cast<const char *>(W) + (size_t)row0 * K * (BF ? 2 : 4);
    __shared__ int arrive;  // Wave4Sync arrivals of the prologue waves
    if (t == 0) arrive = 0;
    __syncthreads();  // before any load: the waves are just starting

    // 1. activation reads (waves 0..3 own the input elements).  A CU serves
    // its vector memory requests in issue order.  Input-first kernels (QKVG,
    // o_proj, LM head: measured faster so) issue every activation read
    // before any weight load (s_barrier, which waits for no memory), so the
    // input arrives ahead of the CU's weight slice, and stream their weights
    // from waves 4..15 only (a wave stalls at load issue while its SIMD's
    // queue is full, which would hold the prologue back).  gate/up and down
    // (measured faster so) let all 16 waves issue weights at once, the input
    // waves after their activation reads.
    constexpr bool kActFirst = act_first(PRO, EPI);
    constexpr int T0 = kTB - (NTS ? NTS : stream_threads(PRO, EPI));
    static_assert(T0 == 0 || T0 == kT || T0 == 2 * kT, "stream threads: 1024, 768 or 512");
    Prologue<C, K, PRO> pro;
    if (t < kT) pro.load(src);
    // QKVG workgroup j < 16: row j of the tiny a|b projection (a_h for
    // j = h, b_h for j = 8 + h), half-beat t of it on threads t < 128,
    // needed right after the input is built.  (BF16 contracts read the BF16
    // copy: they require BF16-exact weights, so its values are the FP32
    // row's and the workgroup streams 4 KB, not 8 KB, beyond its weight rows.)
    const bool ab_blk = (EPI == EPI_QKVG) && blockIdx.x < 2 * kNH;
    constexpr int ABW = BF ? 2 : 4;
    u32x4 abw[ABW];
    if (ab_blk && t < Hb<kH>::HB) {
        const u32x4 *src4 = BF ? reinterpret_cast<const u32x4 *>(ep.ab16 + (size_t)blockIdx.x * kH + t * 16)
                               : reinterpret_cast<const u32x4 *>(ep.aux + kAuxAB + (size_t)blockIdx.x * kH + t * 16);
#pragma unroll
        for (int q = 0; q < ABW; ++q) abw[q] = src4[q];
    }
    // QKVG extras, read with the activations, ahead of the weight stream:
    // the conv tails and taps of each q/k/v row (its owner lane).  (Read
    // behind the weight loads, they returned after the CU's first weight
    // items, and the compiler's wait for the tails, placed where it widens
    // them, held the prologue waves 0..1 back by about 2 us.)
    const bool owner = wave < CHW && (t & 3) == 0 && (t >> 2) < CR;
    uint16_t tail_b[3] = {0, 0, 0};        // BF16 contracts: the tails' BF16 bits
    float tail_f[3] = {0.0f, 0.0f, 0.0f};  // FP32 contract: FP32 tails
    f32x4 taps = {0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (EPI == EPI_QKVG) {
        const int r = row0 + (t >> 2);
        if (owner && r < 3 * kH) {
            const int kind = r / kH, ch = r - kind * kH;
            if constexpr (BF) {
                const uint16_t *tl = reinterpret_cast<const uint16_t *>(ep.tails + (size_t)kind * kTailStripe);
                tail_b[0] = tl[ch];
                tail_b[1] = tl[kH + ch];
                tail_b[2] = tl[2 * kH + ch];
            } else {
                const float *tl = ep.tails + (size_t)kind * kTailStripe;
                tail_f[0] = tl[ch];
                tail_f[1] = tl[kH + ch];
                tail_f[2] = tl[2 * kH + ch];
            }
            taps = *reinterpret_cast<const f32x4 *>(ep.aux + kAuxConv + ((size_t)kind * kH + ch) * 4);
        }
    }

    if constexpr (kActFirst) __builtin_amdgcn_s_barrier();

    // 2. the weight stream
    // non-temporal weight loads, except in the LM head (measured: plain
    // loads are 1-2 us faster there, and slower in every per-layer GEMV)
    WStream<K, ROWS, C, D, T0, EPI != EPI_LM> ws;
    if (t >= T0) ws.prime(wblk);

    // 3. the input vector in LDS and the fast-path verdict: waves 0..3 build
    // it (synchronising only among themselves); the other waves, once their
    // loads are issued, wait for the prologue's last arrival.
    // 4. the products, in each branch (waves 0..3 take part in gate/up and
    // down).  Where the two branches met before the products, the
    // compiler's wait for a stream wave's first item became a wait for all
    // of its primed items (the prologue branch holds stores and loads whose
    // count it cannot follow); inside the branch it waits item by item.
    const auto products = [&](bool f) __attribute__((always_inline)) {
        if (f) ws.template run<true>(xs, part);
        else ws.template run<false>(xs, part);
    };
    bool fast;
    if (t < kT) {
        // the epilogue's expf table into LDS (a lookup in global memory at
        // the epilogue costs a memory round trip on the kernel's serial
        // tail); the products' barrier makes it visible
        if constexpr (kExpTab) fill_exp2_lds_imm(exp2_lds);
        Wave4Sync sync{&arrive, src.err};
        if constexpr (BF) fast = pro.finish_bf16(src, wi, xs, scratch, bcast, red, sync);
        else fast = pro.finish_fp32(src, reinterpret_cast<float *>(xs), scratch, bcast, sync);
        phase_stamp<ST>(src.stamps, blockIdx.x, 1);
        if constexpr (EPI == EPI_QKVG) {
            if (ab_blk) {
                // a_h or b_h while the weights stream (gdn_gemv_tiny_ab):
                // FP32 products x * w, tree16 per half-beat; then wave 3 runs
                // acc = (acc + tree16(lo)) + tree16(hi) per beat and rounds
                // it (the recurrence turns a_h, b_h into beta_h, decay_h)
                if (t < Hb<kH>::HB) {
                    uint32_t xv[16];
                    lds_load16u(xs + t * 16, xv);
                    float p[16];
                    if constexpr (BF) {
                        const uint32_t wv[8] = {abw[0].x, abw[0].y, abw[0].z, abw[0].w,
                                                abw[1].x, abw[1].y, abw[1].z, abw[1].w};
#pragma unroll
                        for (int i = 0; i < 8; ++i) {
                            p[2 * i] = lane_word_value(xv[2 * i], 0) * u2f(wv[i] << 16);
                            p[2 * i + 1] = lane_word_value(xv[2 * i + 1], 1) * u2f(wv[i] & 0xffff0000u);
                        }
                    } else {
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            p[4 * q + 0] = u2f(xv[4 * q + 0]) * u2f(abw[q].x);
                            p[4 * q + 1] = u2f(xv[4 * q + 1]) * u2f(abw[q].y);
                            p[4 * q + 2] = u2f(xv[4 * q + 2]) * u2f(abw[q].z);
                            p[4 * q + 3] = u2f(xv[4 * q + 3]) * u2f(abw[q].w);
                        }
                    }
                    abpart[t] = tree16(p);
                }
                sync();
                if (t == 3 * 64) {
                    float acc = 0.0f;
                    for (int j = 0; j < Hb<kH>::NB; ++j) acc = (acc + abpart[2 * j]) + abpart[2 * j + 1];
                    ep.ab[blockIdx.x] = R<C>(acc);
                }
            }
        }
        if constexpr (!kActFirst && T0 == 0) products(fast);
    } else {
        if constexpr (BF) {
            wait_count(&arrive, 4 * Prologue<C, K, PRO>::kSyncs, src.err);
            fast = decide_fast(red, wi);
        } else {
            wait_count(&arrive, 4 * Prologue<C, K, PRO>::kSyncsFp32, src.err);
            fast = false;
        }
        if (t >= T0) products(fast);
    }
    __syncthreads();
    phase_stamp<ST>(src.stamps, blockIdx.x, 2);
    if (wave < CHW) {
        const float y = chain_rows<K, CR>(part);
        float conv_out = 0.0f;  // QKVG: the row's conv + SiLU output (owner lanes)
        if (owner) {
            const int rr = t >> 2;  // row within the workgroup
            const int r = row0 + rr;
            if constexpr (EPI == EPI_RAW) {
                ep.y[r] = y;
            } else if constexpr (EPI == EPI_STORE) {
                ep.y[r] = R<C>(y);
            } else if constexpr (EPI == EPI_QKVG) {
                const float yv = R<C>(y);
                if (r < 3 * kH) {
                    // causal conv over [t0, t1, t2, x] + SiLU; tails shift to [t1, t2, x]
                    const int kind = r / kH, ch = r - kind * kH;
                    float t0, t1, t2;
                    if constexpr (BF) {
                        uint16_t *tl = reinterpret_cast<uint16_t *>(ep.tails + (size_t)kind * kTailStripe);
                        t0 = bf16_bits_to_f32(tail_b[0]);
                        t1 = bf16_bits_to_f32(tail_b[1]);
                        t2 = bf16_bits_to_f32(tail_b[2]);
                        tl[ch] = tail_b[1];
                        tl[kH + ch] = tail_b[2];
                        tl[2 * kH + ch] = (uint16_t)(f2u(yv) >> 16);
                    } else {
                        float *tl = ep.tails + (size_t)kind * kTailStripe;
                        t0 = tail_f[0];
                        t1 = tail_f[1];
                        t2 = tail_f[2];
                        tl[ch] = t1;
                        tl[kH + ch] = t2;
                        tl[2 * kH + ch] = yv;
                    }
                    const float s = t0 * taps.x + t1 * taps.y + t2 * taps.z + yv * taps.w;
                    conv_out = R<C>(silu_ref(s, Exp2Lds{exp2_lds}));
                    ep.y[r] = conv_out;
                } else {
                    ep.y2[r - 3 * kH] = yv;
                    ep.y3[r - 3 * kH] = sigmoid_ref(yv, Exp2Lds{exp2_lds});
                }
            } else if constexpr (EPI == EPI_SWIGLU) {
                ybuf[rr] = R<C>(y);
            } else {
                ep.y[r] = y;  // LM: FP32 logits (no rounding point)
                ybuf[rr] = y;
            }
        }
        if constexpr (EPI == EPI_QKVG && BF) {
            // q and k rows: each wave's 16 rows reduced in the tree order of
            // gdn_tree_reduce_256 (its lower four levels) for the recurrence's
            // L2 norms.  Row r sits in the lanes of quad r % 16; the owner's
            // square goes to its quad, then the half-row and row mirrors and
            // the 16- and 32-lane swaps pair rows (2i, 2i+1), then pairs of
            // pairs, and so on (the sums of an XOR butterfly).
            if (row0 < 2 * kH) {
                const auto add = [](uint32_t a, uint32_t b) { return f2u(u2f(a) + u2f(b)); };
                uint32_t v = f2u(conv_out * conv_out);
                v = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x00, 0xf, 0xf, false);  // quad lane 0
                v = add(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x141, 0xf, 0xf, false));
                v = add(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x140, 0xf, 0xf, false));
                const int lane = t & 63;
                const auto s16 = __builtin_amdgcn_permlane16_swap((int)v, (int)v, false, false);
                v = add(v, (uint32_t)(((lane >> 4) & 1) ? s16[0] : s16[1]));
                const auto s32 = __builtin_amdgcn_permlane32_swap((int)v, (int)v, false, false);
                v = add(v, (uint32_t)((lane >> 5) ? s32[0] : s32[1]));
                if (lane == 0) ep.qk_part[2 * blockIdx.x + wave] = u2f(v);
            }
        }
    }

    // 5. workgroup epilogues over all rows
    if constexpr (EPI == EPI_SWIGLU) {
        __syncthreads();
        if (t < ROWS / 2) {
            const float g = ybuf[t], u = ybuf[t + ROWS / 2];
            ep.y[blockIdx.x * (ROWS / 2) + t] = R<C>(silu_ref(g, Exp2Lds{exp2_lds}) * u);
        }
    } else if constexpr (EPI == EPI_LM) {
        // the workgroup's argmax in row order: strict '>' within a lane's
        // rows, then a merge that keeps the larger value and, on ties, the
        // lower index (NaN never wins)
        __syncthreads();
        if (wave == 0) {
            float best = -3.402823466e38f;
            int idx = 0;
            for (int i = t; i < ROWS; i += 64) {
                const float v = ybuf[i];
                if (v > best) {
                    best = v;
                    idx = row0 + i;
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
            if (t == 0) {
                ep.part_val[blockIdx.x] = best;
                ep.part_idx[blockIdx.x] = idx;
            }
        }
    }

    // the product-counter copy of the GEMV input (debug: off in the timed
    // path, where xdump is null); xs is unchanged since the prologue.  At
    // the end, because the compiler cannot count this loop's stores: any
    // load whose value is used after it would wait for every outstanding
    // memory operation of the wave (earlier, that held the stream waves'
    // first products until all their primed items had arrived).
    if (src.xdump != nullptr && blockIdx.x == 0) {
        for (int i = t; i < K; i += kTB) src.xdump[i] = xs[i];
        if (t == 0) src.xdump[K] = fast ? 1u : 0u;
    }
    if constexpr (ST) {
        __syncthreads();
        phase_stamp<ST>(src.stamps, blockIdx.x, 3);
    }
}

// Second argmax stage over the LM head's per-block results, which are in
// index order: strict '>' within a thread's increasing indices, then a
// merge that keeps the larger value and, on ties, the lower index.
template <bool ST>
__global__ __launch_bounds__(kT) void k_argmax(const float *__restrict__ part_val,
                                               const int *__restrict__ part_idx, int n,
                                               int *__restrict__ tok_out, uint64_t *stamps) {
    phase_stamp<ST>(stamps, 0, 0);
    __shared__ float bv[4];
    __shared__ int bi[4];
    float best = -3.402823466e38f;
    int idx = 0;
    for (int i = threadIdx.x; i < n; i += kT) {
        const float v = part_val[i];
        if (v > best) {
            best = v;
            idx = part_idx[i];
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
        phase_stamp<ST>(stamps, 0, 3);
        tok_out[0] = idx;  // host-mapped: the step's completion signal
    }
}

// One workgroup per (16 state columns, head): grid (kHD / CB, kNH), state
// in the tiled layout.  beta_h and decay_h are evaluated from the QKVG
// kernel's a_h and b_h in every workgroup of head h.  PRE: the q/k sums of squares come from the QKVG
// kernel and the output norm's chunk sums go to o_sum (BF16 contracts).
template <int C, int CB, bool PRE, bool ST = false>
__global__ __launch_bounds__(kT) void k_recur(const float *__restrict__ qp,
                                              const float *__restrict__ kp,
                                              const float *__restrict__ vp, ScalarsFromAB scal,
                                              const float *__restrict__ qk_part,
                                              void *__restrict__ state, float *__restrict__ attn,
                                              float *__restrict__ o_sum, uint64_t *stamps) {
    recur_block<C, CB, true, PRE, PRE, ST>(qp, kp, vp, scal, qk_part, state, attn, o_sum, blockIdx.y,
                                           blockIdx.x * CB, stamps, blockIdx.y * gridDim.x + blockIdx.x);
}

// out = R(a + b) over the hidden vector (layer output for the layer hook).
template <int C>
__global__ __launch_bounds__(kT) void k_resadd(const float *__restrict__ a,
                                               const float *__restrict__ b,
                                               float *__restrict__ out) {
    for (int i = threadIdx.x; i < kH; i += kT) out[i] = R<C>(a[i] + b[i]);
}

}  // namespace gdn

// ===================================================================== engine

using namespace gdn;

// Per-matrix column counts of the native multiplier's special inputs, for
// the product counters: colspec[k] = rows whose weight in column k has a zero
// or all-ones exponent, colsub[k] = rows whose weight there is subnormal.
struct ColCounts {
    std::vector<uint32_t> spec, sub;
};

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
    uint16_t *ab16 = nullptr;  // [layers][16][kH]: the a/b rows' BF16 bits
    // persistent state: recurrent [L][8][256 K][256 V] (FP32, or BF16 for
    // REF) and conv tails [L][q,k,v] stripes of kTailStripe floats (BF16
    // payload in the first half for the BF16 contracts)
    void *state = nullptr;
    float *tails = nullptr;
    // activations and step outputs
    float *act = nullptr;
    size_t act_floats = 0;
    float *resid = nullptr, *resid_alt = nullptr, *fhid = nullptr, *qkv = nullptr,
          *gate = nullptr, *sgate = nullptr, *ab = nullptr, *attn = nullptr,
          *ybuf_o = nullptr, *dbuf = nullptr, *hbuf = nullptr, *lm_val = nullptr,
          *xrow = nullptr, *logits = nullptr, *qkpart = nullptr, *osum = nullptr;
    int *lm_idx = nullptr;
    // pinned, mapped, coherent host words: [0] token in, [1] token out (-1
    // until the step's argmax lands), [2] kernel error word
    int *tok_host = nullptr;
    int *tok_map = nullptr;   // the device's address of tok_host
    bool failed = false;      // a step timed out or reported an error
    double timeout_ms = 10000.0;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    bool use_graph = true;
    // the persistent step (gdn_persist.hip): available (weights packed in
    // its stream order, exchange area held), and chosen for captured steps
    bool persist = false;
    bool use_persist = false;
    // phase stamps of every kernel of the step (GDN_GRAPH_STAMPS=1 at init):
    // [node][kStampWGs][kStampSlots], node 5 l + {0 QKVG, 1 recurrence,
    // 2 o_proj, 3 gate/up, 4 down} for layer l, then 5 L the LM head and
    // 5 L + 1 the argmax; null when off
    uint64_t *gstamps = nullptr;
    uint32_t *xbuf = nullptr;
    uint32_t tag0 = 0;
    pst::Params pp{};
    // product counters: GEMV inputs of one step (device, lane words + the
    // fast-path verdict per launch) and the weights' column counts
    uint32_t *xdump = nullptr;
    bool counting = false;
    bool trace_counts = false;    // GDN_COUNTER_TRACE=1: per-slot report on stderr
    std::vector<ColCounts> cols;  // per layer: qkvg, o, gu, down; then the LM head
    // host mirrors for the reference's run-state fields
    GDNRunState *owner = nullptr;
};

constexpr int kStampWGs = 256;                   // slots per node: the widest grid
constexpr int kStampNodes = 5 * kMaxLayers + 2;  // nodes of the largest step
constexpr size_t kStampBytes = (size_t)kStampNodes * kStampWGs * kStampSlots * 8;

namespace {

size_t welem(int contract) { return contract == kFp32 ? 4 : 2; }

uint64_t *node_stamps(GDNEngine *e, int node) {
    return e->gstamps ? e->gstamps + (size_t)node * kStampWGs * kStampSlots : nullptr;
}

float *layer_aux(GDNEngine *e, int l) { return e->aux + (size_t)l * kAuxLayer; }
float *final_norm(GDNEngine *e) { return e->aux + (size_t)e->layers * kAuxLayer; }
float *layer_tails(GDNEngine *e, int l) { return e->tails + (size_t)l * 3 * kTailStripe; }
void *layer_state(GDNEngine *e, int l) {
    const size_t off = (size_t)l * kNH * kHD * kHD;
    if (e->contract == kRef) return static_cast<uint16_t *>(e->state) + off;
    return static_cast<float *>(e->state) + off;
}
size_t state_floats(const GDNEngine *e) { return (size_t)e->layers * kNH * kHD * kHD; }
size_t state_bytes(const GDNEngine *e) { return state_floats(e) * (e->contract == kRef ? 2 : 4); }
size_t tail_floats(const GDNEngine *e) { return (size_t)e->layers * 3 * kTailStripe; }

// The recurrent state's row-major order [heads][256 K][256 V] (.gdnstate)
// <-> the device's tiled order, in which each recurrence workgroup's 256 x
// kCB tile is contiguous (state_index<true, kCB>).
template <class T>
void tile_state(const T *src, T *dst, size_t heads, bool to_tiles) {
    for (size_t h = 0; h < heads; ++h)
        for (int j = 0; j < kHD; ++j)
            for (int c = 0; c < kHD; ++c) {
                const size_t rm = h * kHD * kHD + (size_t)j * kHD + c;
                const size_t tl = h * kHD * kHD + (size_t)(c / kCB) * kHD * kCB + (size_t)j * kCB + (c % kCB);
                if (to_tiles) dst[tl] = src[rm];
                else dst[rm] = src[tl];
            }
}

// Product-counter slots: one per GEMV launch of a step (layer l: 4l QKVG,
// 4l + 1 o_proj, 4l + 2 gate/up, 4l + 3 down; 4L the LM head), each K lane
// words and the fast-path verdict.
constexpr int kDumpStride = kI + 64;
uint32_t *dump_slot(GDNEngine *e, int slot) {
    return e->counting ? e->xdump + (size_t)slot * kDumpStride : nullptr;
}

// Pack rows of BF16-exact FP32 words into the device matrix at `dst`.
// In verify mode upload() downloads the device copy instead and counts the
// bytes that differ from the packing (gdn_validate_weight_shards).
struct Packer {
    int contract;
    std::vector<unsigned char> staging;
    bool verify = false;
    size_t mismatches = 0;
    float min_abs = INFINITY;
    float max_abs = 0.0f;
    int nonfinite = 0;
    size_t filled = 0;  // elements

    void begin(size_t elems) {
        staging.resize(elems * welem(contract));
        min_abs = INFINITY;
        max_abs = 0.0f;
        nonfinite = 0;
        filled = 0;
    }
    void rows(const float *src, size_t n, bool daz = true) {
        float mn, mx;
        int bad;
        if (contract == kFp32) {
            std::memcpy(staging.data() + filled * 4, src, n * 4);
            gdn_scan_fp32(src, n, &mn, &mx, &bad);
        } else {
            uint16_t *d = reinterpret_cast<uint16_t *>(staging.data()) + filled;
            if (daz) {
                gdn_pack_bf16_daz(src, d, n, &mn, &mx, &bad);
            } else {
                for (size_t i = 0; i < n; ++i) {
                    uint32_t b;
                    std::memcpy(&b, src + i, 4);
                    d[i] = (uint16_t)(b >> 16);
                }
                mn = INFINITY;
                mx = 0.0f;
                bad = 0;
            }
        }
        if (mn < min_abs) min_abs = mn;
        if (mx > max_abs) max_abs = mx;
        nonfinite |= bad;
        filled += n;
    }
    // Reorders the staged matrix into the CU-resident GEMV's stream order
    // (stream_piece) for nt stream threads, one workgroup slice of `rows`
    // rows at a time.
    void stream_order(size_t rows, size_t K, int nt) {
        const size_t es = welem(contract), wpi = es;  // 16-byte pieces per 16-element item
        const size_t slice = rows * K * es, nslices = filled * es / slice;
        const int items = (int)(rows * K / 16);
        std::vector<unsigned char> tmp(slice);
        for (size_t b = 0; b < nslices; ++b) {
            unsigned char *sl = staging.data() + b * slice;
            std::memcpy(tmp.data(), sl, slice);
            for (int f = 0; f < items; ++f)
                for (int q = 0; q < (int)wpi; ++q)
                    std::memcpy(sl + 16 * stream_piece(f, q, items, nt, (int)wpi), tmp.data() + 16 * (f * wpi + q), 16);
        }
    }
    int upload(void *dst) {
        return transfer(dst, staging.data(), filled * welem(contract));
    }
    // H2D of `bytes` at `src`, or in verify mode D2H and compare.
    int transfer(void *dst, const void *src, size_t bytes) {
        if (!verify) {
            GDN_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
            return 0;
        }
        std::vector<unsigned char> back(bytes);
        GDN_HIP(hipMemcpy(back.data(), dst, bytes, hipMemcpyDeviceToHost));
        const unsigned char *a = back.data(), *b = static_cast<const unsigned char *>(src);
        for (size_t i = 0; i < bytes; ++i) mismatches += a[i] != b[i];
        return 0;
    }
    WInfo info() const { return WInfo{min_abs, max_abs, nonfinite}; }
};

int check_shape(const GDNWeightHeader *c) {
    if (c->hidden_size != (uint32_t)kH || c->num_heads != (uint32_t)kNH ||
        c->num_v_heads != (uint32_t)kNH || c->head_dim != (uint32_t)kHD ||
        c->intermediate_size != (uint32_t)kI || c->conv_size != 4u) {
        gdn_error("gdn: the kernels are built for hidden 2048, 8 heads of 256, intermediate 5632 "
                  "and conv width 4; the model header differs");
        return -1;
    }
    if (c->num_layers < 1 || c->num_layers > (uint32_t)kMaxLayers) {
        std::fprintf(stderr, "gdn: %u layers; the engine takes 1..%d\n", c->num_layers, kMaxLayers);
        return -1;
    }
    if (c->vocab_size == 0 || (c->vocab_size % kCuLmSmall) != 0) {
        std::fprintf(stderr, "gdn: vocabulary %u is not a positive multiple of %d (the LM head's rows per workgroup)\n",
                     c->vocab_size, kCuLmSmall);
        return -1;
    }
    return 0;
}

// Packs the model into the device layout and uploads it; with verify set
// (gdn_validate_weight_shards) compares the device copy with the packing
// instead and returns the number of differing bytes in *mismatches.
int upload_weights(GDNEngine *e, const GDNModel *m, bool verify = false, size_t *mismatches = nullptr) {
    const size_t H = kH, I = kI, V = (size_t)e->vocab, L = (size_t)e->layers;
    const size_t per_layer = 4 * H * H + H * H + 2 * I * H + H * I;
    const size_t total = L * per_layer + 2 * V * H;
    const size_t es = welem(e->contract);
    // stream threads of each matrix's layout: the per-kernel step's, or the
    // persistent step's (which the per-kernel kernels then also stream)
    const auto nts = [e](int pro, int epi) { return e->persist ? pst::kNT : stream_threads(pro, epi); };
    if (!verify) GDN_HIP(hipMalloc(&e->wmem, total * es));
    char *p = static_cast<char *>(e->wmem);
    Packer pk{e->contract, {}};
    pk.verify = verify;
    for (size_t l = 0; l < L; ++l) {
        const GDNLayerWeights &w = m->layers[l];
        pk.begin(4 * H * H);
        pk.rows(w.q_proj, H * H);
        pk.rows(w.k_proj, H * H);
        pk.rows(w.v_proj, H * H);
        pk.rows(w.g_proj, H * H);
        pk.stream_order(kCuQkvg, H, nts(PRO_RESNORM, EPI_QKVG));
        e->w_qkvg[l] = p;
        e->i_qkvg[l] = pk.info();
        if (pk.upload(p)) return -1;
        p += 4 * H * H * es;

        pk.begin(H * H);
        pk.rows(w.o_proj, H * H);
        pk.stream_order(kCuO, H, nts(PRO_ONORM, EPI_STORE));
        e->w_o[l] = p;
        e->i_o[l] = pk.info();
        if (pk.upload(p)) return -1;
        p += H * H * es;

        // gate/up rows interleaved per workgroup: G gate rows, then the
        // matching G up rows
        pk.begin(2 * I * H);
        const size_t G = kCuGu / 2;
        for (size_t blk = 0; blk < I / G; ++blk) {
            pk.rows(w.mlp_gate_proj + blk * G * H, G * H);
            pk.rows(w.mlp_up_proj + blk * G * H, G * H);
        }
        pk.stream_order(kCuGu, H, nts(PRO_RESNORM, EPI_SWIGLU));
        e->w_gu[l] = p;
        e->i_gu[l] = pk.info();
        if (pk.upload(p)) return -1;
        p += 2 * I * H * es;

        pk.begin(H * I);
        pk.rows(w.mlp_down_proj, H * I);
        pk.stream_order(kCuDown, I, nts(PRO_PLAIN, EPI_STORE));
        e->w_down[l] = p;
        e->i_down[l] = pk.info();
        if (pk.upload(p)) return -1;
        p += H * I * es;
    }
    pk.begin(V * H);
    pk.rows(m->lm_head, V * H);
    pk.stream_order((V % kCuLm) == 0 ? kCuLm : kCuLmSmall, H, nts(PRO_RESNORM, EPI_LM));
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
    if (!verify) GDN_HIP(hipMalloc(&e->aux, aux.size() * 4));
    if (pk.transfer(e->aux, aux.data(), aux.size() * 4)) return -1;
    // the a/b rows' top halves (the BF16 values under the BF16 contracts'
    // BF16-exact weights; unused by the FP32 contract)
    std::vector<uint16_t> ab16(L * 2 * kNH * H);
    for (size_t l = 0; l < L; ++l)
        for (size_t i = 0; i < 2 * kNH * H; ++i) {
            uint32_t b;
            std::memcpy(&b, aux.data() + l * kAuxLayer + kAuxAB + i, 4);
            ab16[l * 2 * kNH * H + i] = (uint16_t)(b >> 16);
        }
    if (!verify) GDN_HIP(hipMalloc(&e->ab16, ab16.size() * 2));
    if (pk.transfer(e->ab16, ab16.data(), ab16.size() * 2)) return -1;
    GDN_HIP(hipDeviceSynchronize());
    if (mismatches) *mismatches = pk.mismatches;
    return 0;
}

int alloc_buffers(GDNEngine *e) {
    GDN_HIP(hipMalloc(&e->state, state_bytes(e)));
    GDN_HIP(hipMemset(e->state, 0, state_bytes(e)));
    GDN_HIP(hipMalloc(&e->tails, tail_floats(e) * 4));
    GDN_HIP(hipMemset(e->tails, 0, tail_floats(e) * 4));
    const size_t nblk_lm = (size_t)e->vocab / kCuLmSmall;  // the most LM-head workgroups
    auto up64 = [](size_t n) { return (n + 63) & ~(size_t)63; };  // 256-byte aligned pieces
    const size_t act_floats = 3 * kH + 3 * kH + 2 * kH + 64 + 3 * kH + kI + up64(nblk_lm) + kH +
                              up64((size_t)e->vocab) + 2 * kNH * 16 + kNH * (kHD / 16);
    GDN_HIP(hipMalloc(&e->act, act_floats * 4));
    e->act_floats = act_floats;
    GDN_HIP(hipMemset(e->act, 0, act_floats * 4));
    float *p = e->act;
    e->resid = p; p += kH;
    e->resid_alt = p; p += kH;
    e->fhid = p; p += kH;
    e->qkv = p; p += 3 * kH;
    e->gate = p; p += kH;
    e->sgate = p; p += kH;
    e->ab = p; p += 64;
    e->attn = p; p += kH;
    e->ybuf_o = p; p += kH;
    e->dbuf = p; p += kH;
    e->hbuf = p; p += kI;
    e->lm_val = p; p += up64(nblk_lm);
    e->xrow = p; p += kH;
    e->logits = p; p += up64((size_t)e->vocab);
    e->qkpart = p; p += 2 * kNH * 16;
    e->osum = p; p += kNH * (kHD / 16);
    GDN_HIP(hipMalloc(&e->lm_idx, nblk_lm * sizeof(int)));
    // the step reads its token from and writes its argmax to host memory
    // directly: no copy kernels on a token's path
    GDN_HIP(hipHostMalloc(&e->tok_host, 4 * sizeof(int), hipHostMallocMapped | hipHostMallocCoherent));
    e->tok_host[0] = e->tok_host[1] = e->tok_host[2] = e->tok_host[3] = 0;
    GDN_HIP(hipHostGetDevicePointer(reinterpret_cast<void **>(&e->tok_map), e->tok_host, 0));
    GDN_HIP(hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking));
    GDN_HIP(hipEventCreate(&e->ev0));
    GDN_HIP(hipEventCreate(&e->ev1));
    if (const char *env = std::getenv("GDN_COUNTER_TRACE")) e->trace_counts = env[0] == '1';
    if (const char *env = std::getenv("GDN_KERNEL_WAIT_TIMEOUT_MS")) {
        const double v = std::atof(env);
        if (v > 0.0) e->timeout_ms = v;
    }
    return 0;
}

// The persistent step's kernel arguments (everything but the tag base).
void fill_persist_params(GDNEngine *e) {
    pst::Params &p = e->pp;
    for (int l = 0; l < e->layers; ++l) {
        p.w_qkvg[l] = e->w_qkvg[l];
        p.w_o[l] = e->w_o[l];
        p.w_gu[l] = e->w_gu[l];
        p.w_down[l] = e->w_down[l];
        p.i_qkvg[l] = e->i_qkvg[l];
        p.i_o[l] = e->i_o[l];
        p.i_gu[l] = e->i_gu[l];
        p.i_down[l] = e->i_down[l];
    }
    p.w_lm = e->w_lm;
    p.i_lm = e->i_lm;
    p.w_emb = e->w_emb;
    p.aux = e->aux;
    p.ab16 = e->ab16;
    p.state = e->state;
    p.tails = e->tails;
    p.xbuf = e->xbuf;
    p.logits = e->logits;
    p.fhid = e->fhid;
    p.resid = e->resid;
    p.xrow = e->xrow;
    p.tok = e->tok_map;
    p.layers = e->layers;
    p.eps = e->eps;
    p.tag0 = 0;
    p.stamps = nullptr;
}

XSrc xsrc(GDNEngine *e, const float *a, const float *b, const float *c, const float *w, float *res_out,
          float *aux_out, uint32_t *xdump) {
    XSrc x{};
    x.a = a;
    x.b = b;
    x.c = c;
    x.w = w;
    x.res_out = res_out;
    x.aux_out = aux_out;
    x.err = e->tok_map + 2;
    x.xdump = xdump;
    x.eps = e->eps;
    return x;
}

// k_gemv_cu in the stream order of the engine's weights (the persistent
// step's 512-thread order when the engine has it).
template <int C, int K, int ROWS, int D, int PRO, int EPI>
void launch_gemv(GDNEngine *e, dim3 grid, hipStream_t s, const void *W, WInfo wi, const XSrc &x, const Epi &ep) {
    if constexpr (C == kBf16w) {
        if (e->gstamps) {  // the stamped copy (never with the persistent layout: init refuses both)
            hipLaunchKernelGGL((k_gemv_cu<C, K, ROWS, D, PRO, EPI, 0, true>), grid, dim3(kTB), 0, s, W, wi, x, ep);
            return;
        }
    }
    if constexpr (C != kFp32) {
        if (e->persist) {
            hipLaunchKernelGGL((k_gemv_cu<C, K, ROWS, D, PRO, EPI, pst::kNT>), grid, dim3(kTB), 0, s, W, wi, x, ep);
            return;
        }
    }
    hipLaunchKernelGGL((k_gemv_cu<C, K, ROWS, D, PRO, EPI>), grid, dim3(kTB), 0, s, W, wi, x, ep);
}

// Per-kernel launches.  The QKVG prologue (PRO0) takes the embedding row
// (first layer of a step), the previous layer's residual (res_b = its down
// output), or a caller-given residual (res_b = nullptr).  Every contract uses
// the CU-resident kernels (grids of 256 one-per-CU workgroups).
template <int C, int PRO0>
void launch_qkvg(GDNEngine *e, int l, const float *res_a, const float *res_b, hipStream_t s) {
    float *aux = layer_aux(e, l);
    Epi q{};
    q.y = e->qkv;
    q.y2 = e->gate;
    q.y3 = e->sgate;
    q.aux = aux;
    q.ab16 = e->ab16 + (size_t)l * 2 * kNH * kH;
    q.tails = layer_tails(e, l);
    q.ab = e->ab;
    q.qk_part = e->qkpart;
    XSrc xq = xsrc(e, res_a, res_b, nullptr, aux + kAuxAttnNorm, e->resid, nullptr, dump_slot(e, 4 * l));
    xq.stamps = node_stamps(e, 5 * l);
    if constexpr (PRO0 == PRO_EMBED) {
        xq.emb = e->w_emb;
        xq.tok = e->tok_map;
        xq.vocab = e->vocab;
        xq.aux_out = e->xrow;
    }
    launch_gemv<C, kH, kCuQkvg, Depth<C>::qkvg, PRO0, EPI_QKVG>(e, dim3(4 * kH / kCuQkvg), s, e->w_qkvg[l],
                                                                e->i_qkvg[l], xq, q);
}

template <int C>
void launch_recur(GDNEngine *e, int l, hipStream_t s) {
    const float *aux = layer_aux(e, l);
    const ScalarsFromAB scal{e->ab, e->ab + kNH, aux + kAuxALog, aux + kAuxDtBias};
    if constexpr (C == kBf16w) {
        if (e->gstamps) {
            hipLaunchKernelGGL((k_recur<C, kCB, true, true>), dim3(kHD / kCB, kNH), dim3(kT), 0, s, e->qkv,
                               e->qkv + kH, e->qkv + 2 * kH, scal, e->qkpart, layer_state(e, l), e->attn, e->osum,
                               node_stamps(e, 5 * l + 1));
            return;
        }
    }
    hipLaunchKernelGGL((k_recur<C, kCB, C != kFp32>), dim3(kHD / kCB, kNH), dim3(kT), 0, s, e->qkv,
                       e->qkv + kH, e->qkv + 2 * kH, scal, e->qkpart, layer_state(e, l), e->attn, e->osum, nullptr);
}

template <int C>
void launch_o(GDNEngine *e, int l, hipStream_t s) {
    Epi st{};
    st.y = e->ybuf_o;
    XSrc xo = xsrc(e, e->attn, e->gate, e->sgate, layer_aux(e, l) + kAuxONorm, nullptr, nullptr,
                   dump_slot(e, 4 * l + 1));
    xo.osum = e->osum;
    xo.stamps = node_stamps(e, 5 * l + 2);
    launch_gemv<C, kH, kCuO, Depth<C>::o, PRO_ONORM, EPI_STORE>(e, dim3(kH / kCuO), s, e->w_o[l], e->i_o[l], xo,
                                                                st);
}

template <int C>
void launch_gu(GDNEngine *e, int l, hipStream_t s) {
    Epi sw{};
    sw.y = e->hbuf;
    XSrc xg = xsrc(e, e->resid, e->ybuf_o, nullptr, layer_aux(e, l) + kAuxMlpNorm, e->resid_alt, nullptr,
                   dump_slot(e, 4 * l + 2));
    xg.stamps = node_stamps(e, 5 * l + 3);
    launch_gemv<C, kH, kCuGu, Depth<C>::gu, PRO_RESNORM, EPI_SWIGLU>(e, dim3(2 * kI / kCuGu), s, e->w_gu[l],
                                                                     e->i_gu[l], xg, sw);
}

template <int C>
void launch_down(GDNEngine *e, int l, hipStream_t s) {
    Epi dn{};
    dn.y = e->dbuf;
    XSrc xd = xsrc(e, e->hbuf, nullptr, nullptr, nullptr, nullptr, nullptr, dump_slot(e, 4 * l + 3));
    xd.stamps = node_stamps(e, 5 * l + 4);
    launch_gemv<C, kI, kCuDown, Depth<C>::down, PRO_PLAIN, EPI_STORE>(e, dim3(kH / kCuDown), s, e->w_down[l],
                                                                      e->i_down[l], xd, dn);
}

// LM-head workgroups (= first-stage argmax results) of a contract/vocabulary.
int lm_blocks(const GDNEngine *e) {
    return (e->vocab % kCuLm) == 0 ? e->vocab / kCuLm : e->vocab / kCuLmSmall;
}

template <int C>
void launch_lm(GDNEngine *e, hipStream_t s) {
    Epi lm{};
    lm.y = e->logits;
    lm.part_val = e->lm_val;
    lm.part_idx = e->lm_idx;
    XSrc xl = xsrc(e, e->resid_alt, e->dbuf, nullptr, final_norm(e), e->resid, e->fhid,
                   dump_slot(e, 4 * e->layers));
    xl.stamps = node_stamps(e, 5 * e->layers);
    const dim3 grid(lm_blocks(e));
    if ((e->vocab % kCuLm) == 0) {
        launch_gemv<C, kH, kCuLm, Depth<C>::lm, PRO_RESNORM, EPI_LM>(e, grid, s, e->w_lm, e->i_lm, xl, lm);
    } else {
        hipLaunchKernelGGL((k_gemv_cu<C, kH, kCuLmSmall, Depth<C>::lm_small, PRO_RESNORM, EPI_LM>), grid,
                           dim3(kTB), 0, s, e->w_lm, e->i_lm, xl, lm);
    }
}

void launch_argmax(GDNEngine *e, hipStream_t s) {
    if (e->gstamps)
        hipLaunchKernelGGL(k_argmax<true>, dim3(1), dim3(kT), 0, s, e->lm_val, e->lm_idx, lm_blocks(e),
                           e->tok_map + 1, node_stamps(e, 5 * e->layers + 1));
    else
        hipLaunchKernelGGL(k_argmax<false>, dim3(1), dim3(kT), 0, s, e->lm_val, e->lm_idx, lm_blocks(e),
                           e->tok_map + 1, nullptr);
}

template <int C, int PRO0>
void enqueue_layer(GDNEngine *e, int l, const float *res_a, const float *res_b, hipStream_t s) {
    launch_qkvg<C, PRO0>(e, l, res_a, res_b, s);
    launch_recur<C>(e, l, s);
    launch_o<C>(e, l, s);
    launch_gu<C>(e, l, s);
    launch_down<C>(e, l, s);
}

template <int C>
void enqueue_step_t(GDNEngine *e, hipStream_t s) {
    enqueue_layer<C, PRO_EMBED>(e, 0, nullptr, nullptr, s);
    for (int l = 1; l < e->layers; ++l) enqueue_layer<C, PRO_RESNORM>(e, l, e->resid_alt, e->dbuf, s);
    launch_lm<C>(e, s);
    launch_argmax(e, s);
}

// Kernel kinds timed by gdn_profile_kernels, in output order.
constexpr int kProfKinds = 7;

// Average device time per launch of each kernel kind; each kind is launched
// back to back over every layer's weights, so no launch finds another's
// weights in cache.  Advances the recurrent and conv state.
template <int C>
int profile_t(GDNEngine *e, uint32_t rounds, float *avg_us, uint32_t n) {
    for (uint32_t id = 0; id < n && id < (uint32_t)kProfKinds; ++id) {
        GDN_HIP(hipStreamSynchronize(e->stream));
        GDN_HIP(hipEventRecord(e->ev0, e->stream));
        uint32_t launches = 0;
        for (uint32_t r = 0; r < rounds; ++r) {
            if (id >= 5) {
                if (id == 5) launch_lm<C>(e, e->stream);
                else launch_argmax(e, e->stream);
                ++launches;
                continue;
            }
            for (int l = 0; l < e->layers; ++l, ++launches) {
                switch (id) {
                case 0: launch_qkvg<C, PRO_RESNORM>(e, l, e->resid_alt, e->dbuf, e->stream); break;
                case 1: launch_recur<C>(e, l, e->stream); break;
                case 2: launch_o<C>(e, l, e->stream); break;
                case 3: launch_gu<C>(e, l, e->stream); break;
                default: launch_down<C>(e, l, e->stream); break;
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

void drop_graph(GDNEngine *e) {
    if (e->exec) (void)hipGraphExecDestroy(e->exec);
    if (e->graph) (void)hipGraphDestroy(e->graph);
    e->exec = nullptr;
    e->graph = nullptr;
}

// Waits for the step's argmax to land in host memory (the last kernel
// writes it), with a deadline, then checks the kernels' error word.
int wait_step(GDNEngine *e) {
    const auto t0 = std::chrono::steady_clock::now();
    const auto limit = std::chrono::duration<double, std::milli>(e->timeout_ms);
    unsigned polls = 0;
    while (__atomic_load_n(&e->tok_host[1], __ATOMIC_ACQUIRE) < 0) {
        if ((++polls & 15u) == 0 && std::chrono::steady_clock::now() - t0 > limit) {
            std::fprintf(stderr, "gdn: decode step did not finish within %.0f ms (GDN_KERNEL_WAIT_TIMEOUT_MS)\n",
                         e->timeout_ms);
            e->failed = true;
            return -1;
        }
        __builtin_ia32_pause();
    }
    if (__atomic_load_n(&e->tok_host[2], __ATOMIC_ACQUIRE) != 0) {
        gdn_error("gdn: a kernel's bounded wait ran out; the step's results are not valid");
        e->failed = true;
        return -1;
    }
    return 0;
}

// Token in (host) -> kernels -> token out (host).  Times when asked.
int run_step(GDNEngine *e, int32_t token, int32_t *tok_out, float *inner_ms) {
    if (e->failed) {
        gdn_error("gdn: this run state failed an earlier step");
        return -1;
    }
    if (e->use_graph && !(e->use_persist && !e->counting) && ensure_graph(e) != 0) return -1;
    e->tok_host[0] = token;  // read by layer 0's kernel through tok_map
    __atomic_store_n(&e->tok_host[1], -1, __ATOMIC_RELEASE);
    if (inner_ms) GDN_HIP(hipEventRecord(e->ev0, e->stream));
    if (e->use_graph && e->use_persist && !e->counting) {
        e->pp.tag0 = e->tag0;
        e->tag0 = (e->tag0 + 256u) & 0xffffu;
        if (persist_launch(e->contract, e->pp, e->stream) != 0) return -1;
    } else if (e->use_graph) {
        GDN_HIP(hipGraphLaunch(e->exec, e->stream));
    } else {
        enqueue_step(e, e->stream);
        GDN_HIP(hipGetLastError());
    }
    if (inner_ms) GDN_HIP(hipEventRecord(e->ev1, e->stream));
    if (wait_step(e) != 0) return -1;
    if (tok_out) *tok_out = e->tok_host[1];
    if (inner_ms) {
        GDN_HIP(hipEventSynchronize(e->ev1));
        GDN_HIP(hipEventElapsedTime(inner_ms, e->ev0, e->ev1));
    }
    return 0;
}

// Device -> host copy ordered after the engine's work.
int d2h(GDNEngine *e, void *dst, const void *src, size_t bytes) {
    GDN_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, e->stream));
    GDN_HIP(hipStreamSynchronize(e->stream));
    return 0;
}

int h2d(GDNEngine *e, void *dst, const void *src, size_t bytes) {
    GDN_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, e->stream));
    GDN_HIP(hipStreamSynchronize(e->stream));
    return 0;
}

// Host buffers behind the reference's run-state fields.
struct HostMirror {
    GDNEngine *engine = nullptr;
    float *workspace = nullptr;          // GDN_WS_FLOATS floats
    Beat512 *stripes[GDN_RECURRENT_STATE_PORTS] = {};
};

// The host buffers of every live run state: the reference's state packers
// receive only a stripe array or a head_buffer pointer, which identify
// their run state here.
std::mutex g_mirrors_mu;
std::vector<HostMirror> g_mirrors;

void destroy_engine(GDNEngine *e) {
    if (!e) return;
    // a step that missed its deadline may still be running: let it finish
    // before its buffers go
    if (e->stream) (void)hipStreamSynchronize(e->stream);
    {
        std::lock_guard<std::mutex> lock(g_mirrors_mu);
        for (size_t i = 0; i < g_mirrors.size(); ++i) {
            if (g_mirrors[i].engine != e) continue;
            std::free(g_mirrors[i].workspace);
            for (Beat512 *st : g_mirrors[i].stripes) std::free(st);
            g_mirrors.erase(g_mirrors.begin() + (long)i);
            break;
        }
    }
    drop_graph(e);
    if (e->ev0) (void)hipEventDestroy(e->ev0);
    if (e->ev1) (void)hipEventDestroy(e->ev1);
    if (e->stream) (void)hipStreamDestroy(e->stream);
    (void)hipFree(e->wmem);
    (void)hipFree(e->aux);
    (void)hipFree(e->ab16);
    (void)hipFree(e->state);
    (void)hipFree(e->tails);
    (void)hipFree(e->act);
    (void)hipFree(e->lm_idx);
    (void)hipFree(e->xdump);
    if (e->tok_host) (void)hipHostFree(e->tok_host);
    persist_xbuf_release(e->xbuf);
    (void)hipFree(e->pp.stamps);
    (void)hipFree(e->gstamps);
    delete e;
}

GDNEngine *engine_of(const GDNRunState *state) {
    if (state == nullptr || state->engine == nullptr) {
        gdn_error("gdn: the run state is not initialised");
        return nullptr;
    }
    return state->engine;
}

// Recurrent state [L][8][256][256] FP32 words <-> the device (BF16 bits for
// REF, whose values must then be BF16-exact).
int load_state(GDNEngine *e, const float *rec, size_t floats) {
    const size_t n = state_floats(e);
    if (floats != n) {
        std::fprintf(stderr, "gdn: recurrent state of %zu values given; the model's is %zu\n", floats, n);
        return -1;
    }
    if (e->contract == kRef) {
        const size_t bad = gdn_first_non_bf16(rec, n);
        if (bad != n) {
            gdn_report_non_bf16("REF-contract recurrent state", rec, bad);
            return -1;
        }
        std::vector<uint16_t> b(n), tiles(n);
        for (size_t i = 0; i < n; ++i) {
            uint32_t u;
            std::memcpy(&u, rec + i, 4);
            b[i] = (uint16_t)(u >> 16);
        }
        tile_state(b.data(), tiles.data(), n / (kHD * kHD), true);
        return h2d(e, e->state, tiles.data(), n * 2);
    }
    std::vector<float> tiles(n);
    tile_state(rec, tiles.data(), n / (kHD * kHD), true);
    return h2d(e, e->state, tiles.data(), n * 4);
}

int save_state(GDNEngine *e, float *rec, size_t floats) {
    const size_t n = state_floats(e);
    if (floats != n) {
        std::fprintf(stderr, "gdn: recurrent state buffer of %zu values; the model's is %zu\n", floats, n);
        return -1;
    }
    if (e->contract == kRef) {
        std::vector<uint16_t> tiles(n), b(n);
        if (d2h(e, tiles.data(), e->state, n * 2)) return -1;
        tile_state(tiles.data(), b.data(), n / (kHD * kHD), false);
        for (size_t i = 0; i < n; ++i) {
            const uint32_t u = (uint32_t)b[i] << 16;
            std::memcpy(rec + i, &u, 4);
        }
        return 0;
    }
    std::vector<float> tiles(n);
    if (d2h(e, tiles.data(), e->state, n * 4)) return -1;
    tile_state(tiles.data(), rec, n / (kHD * kHD), false);
    return 0;
}

// .gdnstate conv section [L][q,k,v][W-1][H] <-> the device's tail stripes.
int load_tails(GDNEngine *e, const float *conv, size_t floats) {
    const size_t stripes = (size_t)e->layers * 3, per = 3 * (size_t)kH;
    if (floats != stripes * per) {
        std::fprintf(stderr, "gdn: conv tails of %zu values given; the model's are %zu\n", floats, stripes * per);
        return -1;
    }
    if (e->contract != kFp32) {
        const size_t bad = gdn_first_non_bf16(conv, floats);
        if (bad != floats) {
            gdn_report_non_bf16("BF16-contract conv tail", conv, bad);
            return -1;
        }
    }
    std::vector<float> img(stripes * kTailStripe, 0.0f);
    for (size_t st = 0; st < stripes; ++st) {
        float *dst = img.data() + st * kTailStripe;
        const float *src = conv + st * per;
        if (e->contract == kFp32) {
            std::memcpy(dst, src, per * 4);
        } else {
            uint16_t *d16 = reinterpret_cast<uint16_t *>(dst);
            for (size_t i = 0; i < per; ++i) {
                uint32_t u;
                std::memcpy(&u, src + i, 4);
                d16[i] = (uint16_t)(u >> 16);
            }
        }
    }
    return h2d(e, e->tails, img.data(), img.size() * 4);
}

int save_tails(GDNEngine *e, float *conv, size_t floats) {
    const size_t stripes = (size_t)e->layers * 3, per = 3 * (size_t)kH;
    if (floats != stripes * per) {
        std::fprintf(stderr, "gdn: conv-tail buffer of %zu values; the model's tails are %zu\n", floats,
                     stripes * per);
        return -1;
    }
    std::vector<float> img(stripes * kTailStripe);
    if (d2h(e, img.data(), e->tails, img.size() * 4)) return -1;
    for (size_t st = 0; st < stripes; ++st) {
        const float *src = img.data() + st * kTailStripe;
        float *dst = conv + st * per;
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

// ---- native-product counters of a decode step (counting mode) ----

// The weight matrices of one counter slot, as row blocks of the host model.
struct SlotRows {
    const float *w[4];
    size_t rows[4];
    int n;
    int K;
};

SlotRows slot_rows(const GDNModel *m, int layers, int slot) {
    SlotRows r{};
    if (slot == 4 * layers) {
        r.w[0] = m->lm_head;
        r.rows[0] = m->config.vocab_size;
        r.n = 1;
        r.K = kH;
        return r;
    }
    const GDNLayerWeights &lw = m->layers[slot / 4];
    switch (slot % 4) {
    case 0:
        r.w[0] = lw.q_proj; r.w[1] = lw.k_proj; r.w[2] = lw.v_proj; r.w[3] = lw.g_proj;
        r.rows[0] = r.rows[1] = r.rows[2] = r.rows[3] = kH;
        r.n = 4;
        r.K = kH;
        break;
    case 1:
        r.w[0] = lw.o_proj; r.rows[0] = kH; r.n = 1; r.K = kH;
        break;
    case 2:
        r.w[0] = lw.mlp_gate_proj; r.w[1] = lw.mlp_up_proj;
        r.rows[0] = r.rows[1] = kI; r.n = 2; r.K = kH;
        break;
    default:
        r.w[0] = lw.mlp_down_proj; r.rows[0] = kH; r.n = 1; r.K = kI;
        break;
    }
    return r;
}

int count_step_products(GDNEngine *e, const GDNModel *m) {
    if (e->contract == kFp32) return 0;  // FP32 products: no native multiplier
    const int slots = 4 * e->layers + 1;
    if (e->cols.empty()) {
        e->cols.resize((size_t)slots);
        for (int sl = 0; sl < slots; ++sl) {
            const SlotRows r = slot_rows(m, e->layers, sl);
            ColCounts &c = e->cols[(size_t)sl];
            c.spec.assign((size_t)r.K, 0u);
            c.sub.assign((size_t)r.K, 0u);
            for (int i = 0; i < r.n; ++i)
                gdn_weight_column_counts(r.w[i], r.rows[i], (size_t)r.K, c.spec.data(), c.sub.data());
        }
    }
    std::vector<uint32_t> dump((size_t)slots * kDumpStride);
    if (d2h(e, dump.data(), e->xdump, dump.size() * 4)) return -1;
    uint64_t calls = 0, special = 0, flushed_in = 0, flushed_out = 0, overflow = 0;
    std::vector<uint16_t> xb(kI);
    for (int sl = 0; sl < slots; ++sl) {
        const SlotRows r = slot_rows(m, e->layers, sl);
        const uint32_t *words = dump.data() + (size_t)sl * kDumpStride;
        const ColCounts &c = e->cols[(size_t)sl];
        size_t M = 0;
        for (int i = 0; i < r.n; ++i) M += r.rows[i];
        uint64_t x_special = 0, w_special = 0;
        for (int k = 0; k < r.K; ++k) {
            const uint16_t b = (uint16_t)((k & 1) ? words[k] >> 16 : words[k] & 0xffffu);
            xb[(size_t)k] = b;
            const uint32_t ex = (b >> 7) & 0xffu;
            const bool spec = ex == 0 || ex == 0xffu, sub = ex == 0 && (b & 0x7fu) != 0;
            calls += M;
            special += spec ? M : c.spec[(size_t)k];
            flushed_in += sub ? M : c.sub[(size_t)k];
            x_special += spec;
            w_special += spec ? 0 : c.spec[(size_t)k];
        }
        if (e->trace_counts && (x_special || w_special))
            std::fprintf(stderr, "gdn counters: slot %d (K %d, M %zu): %llu special inputs, %llu special weights "
                         "met by normal inputs, fast path %u\n", sl, r.K, M, (unsigned long long)x_special,
                         (unsigned long long)w_special, words[r.K]);
        if (words[r.K] == 0) {
            // the kernel ran its exact per-product path: count each product's
            // outcome (the fast-path verdict excludes flushes and overflows)
            for (int i = 0; i < r.n; ++i)
                gdn_count_native_outcomes(r.w[i], r.rows[i], (size_t)r.K, xb.data(), &flushed_out, &overflow);
        }
    }
    gdn_stats_add(calls, special, flushed_in, flushed_out, overflow);
    return 0;
}

// Turns the engine's per-step counting on or off to match the process-wide
// switch; the captured graph carries the dump pointers, so it is rebuilt.
int sync_counting(GDNEngine *e) {
    const bool want = gdn_stats_counting() != 0 && e->contract != kFp32;
    if (want == e->counting) return 0;
    if (want && !e->xdump)
        GDN_HIP(hipMalloc(&e->xdump, (size_t)(4 * e->layers + 1) * kDumpStride * 4));
    e->counting = want;
    drop_graph(e);
    return 0;
}

float *g_debug_hidden = nullptr;
float *g_debug_logits = nullptr;

}  // namespace

// ================================================================== C ABI

extern "C" {

int gdn_run_state_init_contract(GDNRunState *state, const GDNModel *model, uint32_t max_tokens,
                                int contract) {
    std::memset(state, 0, sizeof(*state));
    if (max_tokens == 0 || max_tokens > model->config.max_seq_len) {
        std::fprintf(stderr, "gdn_run_state_init: max_tokens %u is outside 1..max_seq_len (%u)\n", max_tokens,
                     model->config.max_seq_len);
        return -1;
    }
    if (contract < kRef || contract > kFp32) {
        std::fprintf(stderr, "gdn_run_state_init: unknown contract %d\n", contract);
        return -1;
    }
    if (check_shape(&model->config) != 0) return -1;
    if (contract != kFp32 && gdn_validate_bf16_exact_weights(model->weight_data, &model->config) != 0) {
        gdn_error("gdn: the BF16 contracts take a BF16-valued checkpoint");
        return -1;
    }
    HostMirror hm;
    hm.workspace = static_cast<float *>(std::aligned_alloc(64, (size_t)GDN_WS_FLOATS * 4));
    bool ok = hm.workspace != nullptr;
    for (int p = 0; ok && p < GDN_RECURRENT_STATE_PORTS; ++p) {
        hm.stripes[p] = static_cast<Beat512 *>(
            std::aligned_alloc(64, (size_t)GDN_RECURRENT_STATE_STRIPE_BF16_BEATS * sizeof(Beat512)));
        ok = hm.stripes[p] != nullptr;
    }
    if (!ok) {
        gdn_error("gdn_run_state_init: host allocation failed");
        std::free(hm.workspace);
        for (Beat512 *st : hm.stripes) std::free(st);
        return -1;
    }
    std::memset(hm.workspace, 0, (size_t)GDN_WS_FLOATS * 4);
    for (Beat512 *st : hm.stripes) std::memset(st, 0, (size_t)GDN_RECURRENT_STATE_STRIPE_BF16_BEATS * 64);
    GDNEngine *e = new GDNEngine();
    e->contract = contract;
    e->layers = (int)model->config.num_layers;
    e->vocab = (int)model->config.vocab_size;
    e->eps = model->config.norm_eps;
    hm.engine = e;
    {
        std::lock_guard<std::mutex> lock(g_mirrors_mu);
        g_mirrors.push_back(hm);
    }
    // the persistent step (opt-in: GDN_PERSIST=1 at init, since it measured
    // slower than the captured graph): BF16 contracts, the 32000-row LM head
    // it is laid out for, a device that holds its grid
    {
        const char *env = std::getenv("GDN_PERSIST");
        const bool on = env != nullptr && env[0] == '1';
        if (on && contract != kFp32 && e->vocab == pst::kWG * pst::kLmRows && persist_supported(contract)) {
            e->xbuf = persist_xbuf_acquire();
            e->persist = e->use_persist = e->xbuf != nullptr;
        }
    }
    if (alloc_buffers(e) != 0 || upload_weights(e, model) != 0) {
        destroy_engine(e);
        return -1;
    }
    if (e->persist) fill_persist_params(e);
    {
        // phase stamps of every step (gdn_test_step_buffers, which = 2 and 3)
        const size_t pbytes = (size_t)pst::kWG * (kMaxLayers + 1) * pst::kStamps * 8;
        const char *gs = std::getenv("GDN_GRAPH_STAMPS");
        bool sok = true;
        if (e->persist && std::getenv("GDN_PERSIST_STAMPS"))
            sok = hipMalloc(&e->pp.stamps, pbytes) == hipSuccess && hipMemset(e->pp.stamps, 0, pbytes) == hipSuccess;
        if (gs != nullptr && gs[0] == '1' &&
            (contract != kBf16w || e->persist || (e->vocab % kCuLm) != 0)) {
            gdn_error("gdn_run_state_init: GDN_GRAPH_STAMPS=1 takes GDN_CONTRACT_BF16W_FP32S, a vocabulary of "
                      "125-row LM-head blocks, and no GDN_PERSIST");
            destroy_engine(e);
            return -1;
        }
        if (sok && gs != nullptr && gs[0] == '1')
            sok = hipMalloc(&e->gstamps, kStampBytes) == hipSuccess &&
                  hipMemset(e->gstamps, 0, kStampBytes) == hipSuccess;
        if (!sok) {
            gdn_error("gdn_run_state_init: phase-stamp buffer allocation failed");
            destroy_engine(e);
            return -1;
        }
    }
    state->engine = e;
    state->workspace = reinterpret_cast<Beat512 *>(hm.workspace);
    state->x = hm.workspace + GDN_WS_OFF_X;
    state->recurrent_state = hm.workspace + GDN_WS_OFF_REC_STATE;
    state->head_buffer = hm.workspace + GDN_WS_OFF_HEAD_BUF;
    for (int p = 0; p < GDN_RECURRENT_STATE_PORTS; ++p)
        state->weight_shards[GDN_RECURRENT_STATE_FIRST_PORT + p] = hm.stripes[p];
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
    return state && state->engine ? state->engine->contract : -1;
}

int gdn_set_graph_mode(GDNRunState *state, int use_graph) {
    GDNEngine *e = engine_of(state);
    if (!e) return -1;
    e->use_graph = use_graph != 0;
    return 0;
}

int gdn_set_persistent(GDNRunState *state, int on) {
    GDNEngine *e = engine_of(state);
    if (!e) return -1;
    if (on && !e->persist) {
        gdn_error("gdn_set_persistent: this run state has no persistent step (contract, vocabulary or device)");
        return -1;
    }
    e->use_persist = on != 0;
    return 0;
}

int gdn_get_persistent(const GDNRunState *state) {
    const GDNEngine *e = state ? state->engine : nullptr;
    if (!e) return -1;
    return (e->use_persist && e->use_graph) ? 1 : 0;
}

int gdn_decode_step_host(const GDNModel *model, GDNRunState *state, const int32_t *token) {
    if (model == nullptr || token == nullptr) {
        gdn_error("gdn_decode_step_host: model and token are required");
        return -1;
    }
    if (*token < 0 || (uint32_t)*token >= model->config.vocab_size) {
        std::fprintf(stderr, "gdn: token %d is outside the vocabulary [0, %u)\n", *token,
                     model->config.vocab_size);
        return -1;
    }
    GDNEngine *e = engine_of(state);
    if (!e || sync_counting(e) != 0) return -1;
    // the reference's host stages the FP32 embedding row in workspace X
    std::memcpy(state->x, model->embeddings + (size_t)*token * kH, (size_t)kH * 4);
    int32_t out = 0;
    if (run_step(e, *token, &out, nullptr) != 0) return -1;
    reinterpret_cast<float *>(state->workspace)[GDN_WS_OFF_X_NORM] = (float)out;  // the token line
    if (g_debug_hidden && d2h(e, g_debug_hidden, e->fhid, (size_t)kH * 4)) return -1;
    if (g_debug_logits && d2h(e, g_debug_logits, e->logits, (size_t)e->vocab * 4)) return -1;
    if (e->counting && count_step_products(e, model) != 0) return -1;
    return 0;
}

int gdn_read_token(const GDNRunState *state, int32_t *token) {
    GDNEngine *e = engine_of(state);
    if (!e) return -1;
    GDN_HIP(hipStreamSynchronize(e->stream));
    *token = e->tok_host[1];
    return 0;
}

int gdn_read_logits(const GDNRunState *state, float *logits, size_t count) {
    GDNEngine *e = engine_of(state);
    if (!e) return -1;
    if (count > (size_t)e->vocab) {
        std::fprintf(stderr, "gdn_read_logits: %zu values asked, the vocabulary has %d\n", count, e->vocab);
        return -1;
    }
    return d2h(e, logits, e->logits, count * 4);
}

int gdn_read_final_hidden(const GDNRunState *state, float *hidden, size_t count) {
    GDNEngine *e = engine_of(state);
    if (!e) return -1;
    if (count > (size_t)kH) {
        std::fprintf(stderr, "gdn_read_final_hidden: %zu values asked, the hidden size is %d\n", count, kH);
        return -1;
    }
    return d2h(e, hidden, e->fhid, count * 4);
}

int gdn_load_recurrent_state(GDNRunState *state, const float *rec, size_t floats) {
    GDNEngine *e = engine_of(state);
    return e ? load_state(e, rec, floats) : -1;
}

int gdn_save_recurrent_state(const GDNRunState *state, float *rec, size_t floats) {
    GDNEngine *e = engine_of(state);
    return e ? save_state(e, rec, floats) : -1;
}

int gdn_load_conv_tails(GDNRunState *state, const float *conv, size_t floats) {
    GDNEngine *e = engine_of(state);
    return e ? load_tails(e, conv, floats) : -1;
}

int gdn_save_conv_tails(const GDNRunState *state, float *conv, size_t floats) {
    GDNEngine *e = engine_of(state);
    return e ? save_tails(e, conv, floats) : -1;
}

// ---- the reference's remaining run-state calls (gdn_model.h:170-210, :274) ----

size_t gdn_weight_shard_beats(const GDNWeightHeader *config) {
    (void)config;
    return 0;
}

size_t gdn_weight_shard_bytes(const GDNWeightHeader *config) {
    (void)config;
    return 0;
}

int gdn_validate_weight_shards(const float *weight_data, const GDNWeightHeader *config, Beat512 *const shards[]) {
    GDNEngine *e = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_mirrors_mu);
        for (auto &m : g_mirrors)
            if (shards != nullptr && m.stripes[0] == shards[GDN_RECURRENT_STATE_FIRST_PORT]) e = m.engine;
    }
    if (!e) {
        gdn_error("gdn_validate_weight_shards: the shard array belongs to no live run state");
        return -1;
    }
    if (config->vocab_size != (uint32_t)e->vocab || config->num_layers != (uint32_t)e->layers) {
        gdn_error("gdn_validate_weight_shards: the header does not describe this run state's model");
        return -1;
    }
    GDNModel view;
    if (gdn_model_wrap(&view, config, weight_data) != 0) return -1;
    size_t bad = 0;
    const int rc = upload_weights(e, &view, /*verify=*/true, &bad);
    std::free(view.layers);
    if (rc != 0) return -1;
    if (bad != 0) {
        std::fprintf(stderr, "gdn_validate_weight_shards: %zu device bytes differ from the packed weights\n", bad);
        return -1;
    }
    return 0;
}

int gdn_scatter_recurrent_state(Beat512 *const state_stripes[], const float *rec, size_t floats) {
    if (state_stripes == nullptr || floats % kHD != 0) {
        gdn_error("gdn_scatter_recurrent_state: no stripes, or the state is not whole 256-value rows");
        return -1;
    }
    GDNEngine *e = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_mirrors_mu);
        for (auto &m : g_mirrors)
            if (m.stripes[0] == state_stripes[0]) e = m.engine;
    }
    // stripes of a run state: the values go to its engine (which checks
    // them for its contract); other stripes are packed only, BF16-exact
    // values required, as the reference's packer does
    if (e != nullptr) {
        if (load_state(e, rec, floats) != 0) return -1;
    } else {
        const size_t bad = gdn_first_non_bf16(rec, floats);
        if (bad != floats) {
            gdn_report_non_bf16("recurrent state", rec, bad);
            return -1;
        }
    }
    gdn_pack_state_stripes(rec, floats / kHD, state_stripes);
    return 0;
}

int gdn_pack_conv_tails_bf16(Beat512 *head_buffer, const float *conv, size_t floats) {
    if (head_buffer == nullptr) {
        gdn_error("gdn_pack_conv_tails_bf16: no head buffer");
        return -1;
    }
    GDNEngine *e = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_mirrors_mu);
        for (auto &m : g_mirrors)
            if (reinterpret_cast<float *>(head_buffer) == m.workspace + GDN_WS_OFF_HEAD_BUF) e = m.engine;
    }
    if (e != nullptr) {
        if (load_tails(e, conv, floats) != 0) return -1;
    } else {
        if (floats != GDN_WSF_HEADBUF) {
            std::fprintf(stderr, "gdn_pack_conv_tails_bf16: %zu values; the workspace holds %u\n", floats,
                         GDN_WSF_HEADBUF);
            return -1;
        }
        const size_t bad = gdn_first_non_bf16(conv, floats);
        if (bad != floats) {
            gdn_report_non_bf16("conv tail", conv, bad);
            return -1;
        }
    }
    gdn_pack_tail_stripes(conv, floats / (3 * (size_t)kH), reinterpret_cast<float *>(head_buffer));
    return 0;
}

int gdn_sync_host_state(GDNRunState *state) {
    GDNEngine *e = engine_of(state);
    if (!e) return -1;
    std::vector<float> rec(state_floats(e)), conv((size_t)e->layers * 9 * kH);
    if (save_state(e, rec.data(), rec.size()) != 0 || save_tails(e, conv.data(), conv.size()) != 0) return -1;
    gdn_pack_state_stripes(rec.data(), rec.size() / kHD, state->weight_shards + GDN_RECURRENT_STATE_FIRST_PORT);
    gdn_pack_tail_stripes(conv.data(), (size_t)e->layers * 3, state->head_buffer);
    return 0;
}

void gdn_set_native_debug_buffers(float *final_hidden, float *logits) {
    g_debug_hidden = final_hidden;
    g_debug_logits = logits;
}

int gdn_run_teacher_forced(GDNRunState *state, const int32_t *tokens, uint32_t n_tokens,
                           uint32_t n_steps, int32_t *argmax_out, float *inner_ms,
                           float *outer_ms) {
    GDNEngine *e = engine_of(state);
    if (!e) return -1;
    if (n_tokens == 0 || tokens == nullptr) {
        gdn_error("gdn_run_teacher_forced: no tokens");
        return -1;
    }
    for (uint32_t i = 0; i < n_tokens; ++i) {
        if (tokens[i] < 0 || tokens[i] >= e->vocab) {
            std::fprintf(stderr, "gdn: token %d (position %u) is outside the vocabulary [0, %d)\n", tokens[i], i,
                         e->vocab);
            return -1;
        }
    }
    if (sync_counting(e) != 0) return -1;
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

int gdn_profile_kernels(GDNRunState *state, uint32_t rounds, float *avg_us, uint32_t n_kinds) {
    GDNEngine *e = engine_of(state);
    if (!e || rounds == 0) return -1;
    switch (e->contract) {
    case kRef: return profile_t<kRef>(e, rounds, avg_us, n_kinds);
    case kBf16w: return profile_t<kBf16w>(e, rounds, avg_us, n_kinds);
    default: return profile_t<kFp32>(e, rounds, avg_us, n_kinds);
    }
}

// ---------------------------------------------------------------- test hooks

int gdn_test_gemv(int contract, const float *W, const float *x, uint32_t M, uint32_t K, float *y) {
    constexpr int kRows = 8;  // rows per workgroup
    if ((K != (uint32_t)kH && K != (uint32_t)kI) || M == 0 || (M % kRows) != 0) {
        gdn_error("gdn_test_gemv: K must be 2048 or 5632 and M a multiple of 8");
        return -1;
    }
    Packer pk{contract, {}};
    pk.begin((size_t)M * K);
    pk.rows(W, (size_t)M * K);
    pk.stream_order(kRows, K, stream_threads(PRO_PLAIN, EPI_RAW));
    void *dW = nullptr;
    float *dx = nullptr, *dy = nullptr;
    GDN_HIP(hipMalloc(&dW, (size_t)M * K * welem(contract)));
    GDN_HIP(hipMalloc(&dx, (size_t)K * 4));
    GDN_HIP(hipMalloc(&dy, (size_t)M * 4));
    if (pk.upload(dW)) return -1;
    GDN_HIP(hipMemcpy(dx, x, (size_t)K * 4, hipMemcpyHostToDevice));
    const WInfo wi = pk.info();
    const dim3 grid(M / kRows);
#define GDN_PLAIN(CC, KK)                                                                                  \
    hipLaunchKernelGGL((k_gemv_cu<CC, KK, kRows, Depth<CC>::o, PRO_PLAIN, EPI_RAW>), grid, dim3(kTB), 0, 0, dW, wi, \
                       xs, ep)
    XSrc xs{};
    xs.a = dx;
    Epi ep{};
    ep.y = dy;
    if (K == (uint32_t)kH) {
        if (contract == kFp32) GDN_PLAIN(kFp32, kH);
        else GDN_PLAIN(kRef, kH);  // the two BF16 contracts share their products
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
        std::vector<uint16_t> sb(nstate), tiles(nstate);
        for (size_t i = 0; i < nstate; ++i) {
            uint32_t u;
            std::memcpy(&u, S + i, 4);
            sb[i] = (uint16_t)(u >> 16);
        }
        tile_state(sb.data(), tiles.data(), n_heads, true);
        GDN_HIP(hipMemcpy(dS, tiles.data(), nstate * 2, hipMemcpyHostToDevice));
    } else {
        std::vector<float> tiles(nstate);
        tile_state(S, tiles.data(), n_heads, true);
        GDN_HIP(hipMemcpy(dS, tiles.data(), nstate * 4, hipMemcpyHostToDevice));
    }
    const dim3 grid(kHD / kCB, n_heads), block(kT);
    for (uint32_t s = 0; s < n_steps; ++s) {
        const size_t ov = (size_t)s * n_heads * kHD, os = (size_t)s * n_heads;
        const ScalarsFromAB scal{da + os, db + os, dal + os, ddt + os};
#define GDN_REC(CC)                                                                                       \
    hipLaunchKernelGGL((k_recur<CC, kCB, false>), grid, block, 0, 0, dq + ov, dk + ov, dv + ov, scal, nullptr, \
                       dS, dout + ov, nullptr, nullptr)
        if (contract == kRef) GDN_REC(kRef);
        else if (contract == kBf16w) GDN_REC(kBf16w);
        else GDN_REC(kFp32);
#undef GDN_REC
    }
    GDN_HIP(hipGetLastError());
    GDN_HIP(hipDeviceSynchronize());
    GDN_HIP(hipMemcpy(o, dout, nv * 4, hipMemcpyDeviceToHost));
    if (contract == kRef) {
        std::vector<uint16_t> sb(nstate), tiles(nstate);
        GDN_HIP(hipMemcpy(tiles.data(), dS, nstate * 2, hipMemcpyDeviceToHost));
        tile_state(tiles.data(), sb.data(), n_heads, false);
        for (size_t i = 0; i < nstate; ++i) {
            const uint32_t u = (uint32_t)sb[i] << 16;
            std::memcpy(S + i, &u, 4);
        }
    } else {
        std::vector<float> tiles(nstate);
        GDN_HIP(hipMemcpy(tiles.data(), dS, nstate * 4, hipMemcpyDeviceToHost));
        tile_state(tiles.data(), S, n_heads, false);
    }
    float *bufs[] = {dq, dk, dv, da, db, dal, ddt, dout};
    for (float *p : bufs) GDN_HIP(hipFree(p));
    GDN_HIP(hipFree(dS));
    return 0;
}

int gdn_test_step_buffers(const GDNRunState *state, int which, void *out, size_t bytes) {
    GDNEngine *e = engine_of(state);
    if (!e || out == nullptr) return -1;
    if (which == 0) {
        if (e->xbuf == nullptr) {
            gdn_error("gdn_test_step_buffers: this run state has no persistent step");
            return -1;
        }
        return d2h(e, out, e->xbuf, std::min(bytes, (size_t)pst::XWORDS * 4));
    }
    if (which == 1) return d2h(e, out, e->act, std::min(bytes, e->act_floats * 4));
    if (which == 2 && e->pp.stamps)
        return d2h(e, out, e->pp.stamps, std::min(bytes, (size_t)pst::kWG * (kMaxLayers + 1) * pst::kStamps * 8));
    if (which == 3 && e->gstamps) return d2h(e, out, e->gstamps, std::min(bytes, kStampBytes));
    gdn_error("gdn_test_step_buffers: which is 0 (exchange area), 1 (activations), 2 (persistent-step stamps, "
              "GDN_PERSIST_STAMPS=1 at init) or 3 (per-kernel step stamps, GDN_GRAPH_STAMPS=1 at init)");
    return -1;
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
#define GDN_LAYER(CC)                                                                         \
    do {                                                                                      \
        enqueue_layer<CC, PRO_RESNORM>(e, (int)layer, din, nullptr, e->stream);                 \
        hipLaunchKernelGGL((k_resadd<CC>), dim3(1), dim3(kT), 0, e->stream, e->resid_alt, e->dbuf, \
                           e->resid);                                                         \
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

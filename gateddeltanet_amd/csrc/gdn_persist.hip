// gdn_persist.hip -- the persistent decode step of libgdn_amd.so (BF16
// contracts): one cooperative launch of 256 one-per-CU workgroups x 512
// threads runs a whole token, token id in -> argmax token id out.
//
// Why one launch.  The per-kernel step (gdn_engine.hip) pays a kernel
// boundary of about 1.6 us at each of its 122 launches, and every kernel
// then waits 1.6-3.4 us for its input while its first weight requests queue:
// HBM idles at every boundary.  Here each workgroup owns the same weight
// slices as the per-kernel step (32 QKVG rows, 8 o_proj rows, 22 + 22
// gate/up rows, 8 down rows, 125 LM-head rows) and streams them through a
// ring of kD items per thread that runs ahead across stage boundaries: while
// a stage waits for its input, the weights of this stage and the next are
// already in flight.
//
// How stages hand over.  A CU returns vector loads in issue order, so a
// vector read of another workgroup's output would queue behind the weight
// ring (measured: 3.0 us one-way under a full stream, 0.7 us idle).  Scalar
// loads take a separate path (1.4 us one-way under the same stream).  Every
// value one workgroup hands another is therefore a tagged 32-bit word
// ((tag << 16) | 16-bit payload) in uncached memory, written with a vector
// store and read with scalar loads (s_load_dwordx16 ... glc, 64 bytes); a
// reader retries a line until every word carries the current tag.  No flags,
// fences or resets.  Measured: all 256 workgroups receive 2048 values 2.1 us
// after the last producer's store, 5632 values 4.2 us, with or without the
// weight stream.
//
// Per layer l (rows as in gdn_engine.hip; every operator's arithmetic is the
// per-kernel step's, so results are bit-identical):
//   QKVG    input R(res + y_down) (layer 0: the embedding row), RMSNorm;
//           products; conv + SiLU, tails, gate; q/k partial squares; a/b
//           rows                                     -> q k v g, qk_part, a b
//   recur   workgroups 0..127, waves 0..3: one head x 16 columns, state
//           tile loaded during the previous layer    -> o, chunk sums
//   o_proj  output norm x gate (sigmoid(g) here), products -> y_o
//   gate/up R(res + y_o), RMSNorm, products, SwiGLU  -> h
//   down    products                                 -> y_down
// then the LM head (FP32 logits, per-workgroup argmax) and workgroup 0's
// merge, which writes the token to mapped host memory.
//
// Every residual stream value lives in every workgroup's LDS (each computes
// the same R(res + y) for all 2048 elements), so only stage outputs cross.
//
// Waits are bounded by time (about 0.1 s each): a wait that runs out sets
// the run's error word and the step's abort word, and every later wait of
// every workgroup returns at once, so the grid always drains.
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>

#include <cstdio>
#include <mutex>
#include <vector>

#include "gdn_amd.h"
#include "gdn_device.h"
#include "gdn_gemv.h"
#include "gdn_internal.h"
#include "gdn_persist.h"

namespace gdn {
namespace pst {

constexpr int kD = 4;          // ring depth: items in flight per thread (divides kSlots, kSlotsLm)
constexpr int kSlots = 28;     // ring slots per layer
constexpr int kSlotsLm = 32;   // ring slots of the LM head
constexpr int kHB = kH / 16;   // half-beats per row at K = 2048
constexpr uint64_t kWaitTicks = 10000000;  // 0.1 s of the 100 MHz real-time counter

// Stages and their ring slots within a layer: QKVG 0..7, o_proj 8..9,
// gate/up 10..20, down 21..26 (the last half full), 27 none.
enum { SQ = 0, SO = 1, SG = 2, SD = 3, SN = 4, SL = 5 };
constexpr int stage_of(int s) { return s < 8 ? SQ : s < 10 ? SO : s < 21 ? SG : s < 27 ? SD : SN; }
constexpr int first_slot(int st) { return st == SQ ? 0 : st == SO ? 8 : st == SG ? 10 : st == SD ? 21 : 27; }
constexpr int rows_of(int st) {
    return st == SQ ? kCuQkvg : st == SO ? kCuO : st == SG ? kCuGu : st == SD ? kCuDown : st == SL ? kLmRows : 0;
}
constexpr int k_of(int st) { return st == SD ? kI : kH; }
constexpr int items_of(int st) { return rows_of(st) * (k_of(st) / 16); }
static_assert(items_of(SQ) == 8 * kNT && items_of(SO) == 2 * kNT, "QKVG: slots 0..7, o_proj: 8..9");
static_assert(items_of(SG) == 11 * kNT, "gate/up: slots 10..20");
static_assert(items_of(SD) > 5 * kNT && items_of(SD) <= 6 * kNT, "down: slots 21..26");
static_assert(items_of(SL) > 31 * kNT && items_of(SL) <= kSlotsLm * kNT, "LM head: 32 slots");
static_assert(kSlots % kD == 0 && kSlotsLm % kD == 0, "ring index of a slot is slot % kD everywhere");

__device__ __forceinline__ uint64_t rt_now() { return __builtin_amdgcn_s_memrealtime(); }

// ------------------------------------------------------------ exchange words

__device__ __forceinline__ uint32_t tag_of(uint32_t tag0, int l, int kind) {
    return (tag0 + 8u * (uint32_t)l + (uint32_t)kind) & 0xffffu;
}

// One word, written by this lane (vector store at system scope: it reaches
// memory without waiting for anything else).
__device__ __forceinline__ void xput(uint32_t *p, uint32_t tag, uint32_t payload16) {
    __hip_atomic_store(p, (tag << 16) | (payload16 & 0xffffu), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Scalar loads of 1, 16 or 64 words at a wave-uniform address; glc: past the
// scalar cache (the area is uncached, so memory holds the only copy).
__device__ __forceinline__ uint32_t sload1(const uint32_t *p) {
    uint32_t v;
    asm volatile("s_load_dword %0, %1, 0x0 glc\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(p) : "memory");
    return v;
}

typedef uint32_t u32x16 __attribute__((ext_vector_type(16)));

#define GDN_WL(src, L) asm volatile("v_writelane_b32 %0, %1, %2" : "+v"(v) : "s"(src), "i"(L))

// Words p[0..63] into lanes 0..63.
__device__ __forceinline__ uint32_t sload64(const uint32_t *p) {
    u32x16 a, b, c, d;
    asm volatile(
        "s_load_dwordx16 %0, %4, 0x0 glc\n\t"
        "s_load_dwordx16 %1, %4, 0x40 glc\n\t"
        "s_load_dwordx16 %2, %4, 0x80 glc\n\t"
        "s_load_dwordx16 %3, %4, 0xc0 glc\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&s"(a), "=&s"(b), "=&s"(c), "=&s"(d)
        : "s"(p)
        : "memory");
    uint32_t v = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) GDN_WL(a[i], i);
#pragma unroll
    for (int i = 0; i < 16; ++i) GDN_WL(b[i], 16 + i);
#pragma unroll
    for (int i = 0; i < 16; ++i) GDN_WL(c[i], 32 + i);
#pragma unroll
    for (int i = 0; i < 16; ++i) GDN_WL(d[i], 48 + i);
    return v;
}

// Words p[0..15] into lanes 0..15 (other lanes 0).
__device__ __forceinline__ uint32_t sload16(const uint32_t *p) {
    u32x16 a;
    asm volatile("s_load_dwordx16 %0, %1, 0x0 glc\n\ts_waitcnt lgkmcnt(0)" : "=&s"(a) : "s"(p) : "memory");
    uint32_t v = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) GDN_WL(a[i], i);
    return v;
}
#undef GDN_WL

// A workgroup's view of the step's failure state: once any wait has run out
// (here or in another workgroup: the abort word), waits return at once.
struct Ctl {
    uint32_t *abort_word;
    int *err;
    uint32_t abort_val;
    bool dead;

    // The stores complete before the wave goes on, so the abort word is in
    // memory before any later word this workgroup writes (workgroup 0 checks
    // it after the last exchange, before it writes the token).
    __device__ __forceinline__ void fail() {
        if ((threadIdx.x & 63) == 0) {
            __hip_atomic_store(abort_word, abort_val, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        dead = true;
    }
};

// The wave's NW words at p (NW = 64: lane i gets word i; NW = 16: lanes
// 0..15) once all of them carry `tag`; returns the 16-bit payloads.
template <int NW>
__device__ __forceinline__ uint32_t xget(const uint32_t *p, uint32_t tag, Ctl &c) {
    static_assert(NW == 64 || NW == 16, "4 lines or 1");
    const int lane = threadIdx.x & 63;
    const uint32_t want = tag << 16;
    uint32_t v = 0;
    if (c.dead) return 0;
    const uint64_t t0 = rt_now();
    for (int it = 0;; ++it) {
        v = NW == 64 ? sload64(p) : sload16(p);
        const bool ok = (NW == 16 && lane >= 16) || ((v ^ want) & 0xffff0000u) == 0;
        if (__builtin_amdgcn_ballot_w64(!ok) == 0) break;
        if ((it & 15) == 15) {
            if (sload1(c.abort_word) == c.abort_val) {
                c.dead = true;
                break;
            }
            if (rt_now() - t0 > kWaitTicks) {
                c.fail();
                break;
            }
        }
    }
    return v & 0xffffu;
}

// FP32 value from the payloads of two adjacent lanes (low half in the even
// lane); valid in the even lane.
__device__ __forceinline__ float join_halves(uint32_t pay) {
    const uint32_t hi = (uint32_t)__builtin_amdgcn_mov_dpp((int)pay, 0xB1, 0xf, 0xf, false);  // lane ^ 1
    return u2f((hi << 16) | (pay & 0xffffu));
}

// ------------------------------------------------------------------- LDS

struct Lds {
    alignas(16) float res[kH];                      // the residual stream (same in every workgroup)
    alignas(16) uint32_t xs[kI];                    // GEMV input lane words
    alignas(16) float part[kLmRows * BankLayout<kH>::RSTR];  // bank partials; the recurrence's product tiles
    alignas(16) float y[kH];                        // exchanged stage output (y_down, y_o) or o
    alignas(16) float g[kH];                        // gate g
    alignas(16) float osum[128];                    // output-norm chunk sums
    alignas(16) float nw[2][kH];                    // [0] attention / final norm, [1] MLP norm weights
    alignas(16) float onw[kHD];                     // output-norm weights
    alignas(16) uint32_t abw[kH / 2];               // a/b row (workgroups 0..15), BF16 pairs
    alignas(16) f32x4 taps[kCuQkvg];                // conv taps of the workgroup's q/k/v rows
    alignas(16) uint32_t tails[kCuQkvg][3];         // their tails t0, t1, t2 (BF16 bits)
    alignas(16) float scal[16];                     // a_log[8], dt_bias[8]
    alignas(16) float scratch[kH / 16];
    alignas(16) float bcast[8];
    alignas(16) uint32_t red[8];
    alignas(16) float ybuf[kLmRows + 3];
    alignas(16) float abpart[kHB];
    // recurrence (workgroups 0..127)
    alignas(16) float rq[kHD], rk[kHD], rv[16], rqp[16], rkp[16], rab[2];
    alignas(16) float dl[16], red2[4], bd[2];
    int arrive;
    alignas(16) uint64_t exp2[32];
    alignas(16) float av[kWG];                      // argmax merge (workgroup 0)
    alignas(16) int ai[kWG];
};

// ------------------------------------------------------------------- ring

struct Ring {
    u32x4 v[kD][2];
};

// Item group I of stage st for this thread (stream order, kNT threads): two
// 16-byte nontemporal loads.  Every vector load of the kernel is issued by
// every thread (a thread past a partial group re-reads the group's last
// item): the compiler counts outstanding loads exactly only when none is
// skipped, and a skipped one turns its waits into waits for every load in
// flight.
template <int ST, int I>
__device__ __forceinline__ void load_item(u32x4 (&dst)[2], const char *slice) {
    constexpr int ITEMS = items_of(ST);
    constexpr int FULL = ITEMS / kNT;
    constexpr int SPAN = I < FULL ? kNT : ITEMS - FULL * kNT;
    const int t = (I < FULL) ? (int)threadIdx.x : min((int)threadIdx.x, SPAN - 1);
    const u32x4 *p = reinterpret_cast<const u32x4 *>(slice) + (size_t)kNT * 2 * I + t;
    dst[0] = __builtin_nontemporal_load(p);
    dst[1] = __builtin_nontemporal_load(p + SPAN);
}

// Item group I of stage st: products of the item's 16 weights with the
// input lane words, tree16, into the bank partials.
template <int ST, int I>
__device__ __forceinline__ void mul_item(const u32x4 (&wv)[2], const uint32_t *xs, float *part, uint32_t (&xv)[16],
                                         bool fast) {
    constexpr int K = k_of(ST);
    constexpr int HB = K / 16;
    constexpr int ITEMS = items_of(ST);
    const int f = (int)threadIdx.x + kNT * I;
    if (ITEMS % kNT == 0 || f < ITEMS) {
        const int row = f / HB, hb = f - row * HB;
        if constexpr (kNT % HB != 0) lds_load16u(xs + hb * 16, xv);
        const uint32_t w8[8] = {wv[0].x, wv[0].y, wv[0].z, wv[0].w, wv[1].x, wv[1].y, wv[1].z, wv[1].w};
        if (fast) {
            float p[16];
            uint32_t rbits[8];
            dot8_bf16(w8, xv, rbits);
            dot8_bf16(w8 + 4, xv + 8, rbits + 4);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                p[2 * e] = u2f(rbits[e] << 16);
                p[2 * e + 1] = u2f(rbits[e] & 0xffff0000u);
            }
            part[BankLayout<K>::index(row, hb)] = tree16(p);
        } else {
            // the exact per-product path (inputs outside the fast path's
            // range: rare), one pair of products at a time, each pair added
            // at once (tree16's first level), to bound its registers
            float s8[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                s8[e] = native_exact(w8[e] & 0xffffu, u2f(xv[2 * e] << 16)) +
                        native_exact(w8[e] >> 16, u2f(xv[2 * e + 1]));
                __builtin_amdgcn_sched_barrier(0);
            }
            const float a0 = s8[0] + s8[1], a1 = s8[2] + s8[3], a2 = s8[4] + s8[5], a3 = s8[6] + s8[7];
            part[BankLayout<K>::index(row, hb)] = (a0 + a1) + (a2 + a3);
        }
    }
}

// This workgroup's slice of stage ST's matrix in layer l, read from the
// kernel arguments where it is needed (pointers held across the layer would
// take scalar registers the exchange reads need).
struct Slices {
    const Params *p;
    int l;
};

__device__ __forceinline__ Slices slices_of(const Params &p, int l) { return Slices{&p, l}; }

template <int ST>
__device__ __forceinline__ const char *slice_sel(const Slices &s) {
    const size_t off = (size_t)blockIdx.x * items_of(ST) * 32;
    if constexpr (ST == SQ) return static_cast<const char *>(s.p->w_qkvg[s.l]) + off;
    else if constexpr (ST == SO) return static_cast<const char *>(s.p->w_o[s.l]) + off;
    else if constexpr (ST == SG) return static_cast<const char *>(s.p->w_gu[s.l]) + off;
    else return static_cast<const char *>(s.p->w_down[s.l]) + off;
}

// Slot S of a layer: multiply slot S, then issue slot S + kD of the same
// layer into its registers.  A layer's first kD slots are issued at the top
// of its loop iteration: no load is in flight across the loop's back edge,
// where the register allocator would copy the ring (and a copy of a
// register with a load in flight waits for that load).
template <int S>
__device__ __forceinline__ void proc(Ring &r, const Slices &cur, const uint32_t *xs, float *part,
                                     uint32_t (&xv)[16], bool fast) {
    constexpr int sst = stage_of(S);
    if constexpr (sst != SN) mul_item<sst, S - first_slot(sst)>(r.v[S % kD], xs, part, xv, fast);
    constexpr int N = S + kD;
    if constexpr (N < kSlots) {
        constexpr int st = stage_of(N);
        if constexpr (st != SN) load_item<st, N - first_slot(st)>(r.v[N % kD], slice_sel<st>(cur));
    }
    // one item's products at a time: hoisting later items' work would keep
    // their registers live beside the ring's
    __builtin_amdgcn_sched_barrier(0);
}

// A layer's (or the LM head's) first kD slots.
template <int ST, int I>
__device__ __forceinline__ void prime(Ring &r, const char *slice) {
    if constexpr (I < kD) {
        load_item<ST, I>(r.v[I], slice);
        prime<ST, I + 1>(r, slice);
    }
}

template <int S>
__device__ __forceinline__ void proc_lm(Ring &r, const char *lm, const uint32_t *xs, float *part,
                                        uint32_t (&xv)[16], bool fast) {
    mul_item<SL, S>(r.v[S % kD], xs, part, xv, fast);
    if constexpr (S + kD < kSlotsLm) load_item<SL, S + kD>(r.v[(S + kD) % kD], lm);
    __builtin_amdgcn_sched_barrier(0);
}

template <int S0, int S1>
__device__ __forceinline__ void proc_range(Ring &r, const Slices &cur, const uint32_t *xs, float *part,
                                           uint32_t (&xv)[16], bool fast) {
    if constexpr (S0 <= S1) {
        proc<S0>(r, cur, xs, part, xv, fast);
        proc_range<S0 + 1, S1>(r, cur, xs, part, xv, fast);
    }
}

template <int S0, int S1>
__device__ __forceinline__ void proc_stage(bool fast, Ring &r, const Slices &cur, const uint32_t *xs, float *part) {
    uint32_t xv[16];
    constexpr int K = k_of(stage_of(S0));
    if constexpr (kNT % (K / 16) == 0) lds_load16u(xs + ((int)threadIdx.x % (K / 16)) * 16, xv);
    proc_range<S0, S1>(r, cur, xs, part, xv, fast);
}

template <int S0, int S1>
__device__ __forceinline__ void proc_lm_range(Ring &r, const char *lm, const uint32_t *xs, float *part,
                                              uint32_t (&xv)[16], bool fast) {
    if constexpr (S0 <= S1) {
        proc_lm<S0>(r, lm, xs, part, xv, fast);
        proc_lm_range<S0 + 1, S1>(r, lm, xs, part, xv, fast);
    }
}

// ------------------------------------------------------------ side data

// Per-layer small weights and the recurrent state tile of the next layer,
// issued a stage ahead (they queue behind the ring) and committed to LDS
// (the state stays in registers) once the stage's products are done.
// Every thread issues the same three 16-byte loads; its role picks the
// address (a thread with no role re-reads a valid one):
//   a: attention (LM head: final) norm [4t, 4t+4); m: MLP norm [4t, 4t+4);
//   b: t < 64 output norm [4t, 4t+4); 64..95 conv taps of row t - 64;
//      96..191 the 16 bytes holding tail j = (t - 96) / 32 of row
//      (t - 96) % 32; 192..195 a_log / dt_bias; 256..511 the a/b row
//      (workgroups 0..15)
struct Side {
    f32x4 a = {0.0f, 0.0f, 0.0f, 0.0f};
    f32x4 m = {0.0f, 0.0f, 0.0f, 0.0f};
    u32x4 b = {0u, 0u, 0u, 0u};
};

__device__ __forceinline__ void side_issue(Side &sd, const Params &p, int l, bool lm) {
    static_assert(kNT * 4 == kH, "one f32x4 of each norm per thread");
    const int t = threadIdx.x, w = blockIdx.x;
    const float *aux = p.aux + (size_t)l * kAuxLayer;
    const float *na = lm ? p.aux + (size_t)p.layers * kAuxLayer : aux + kAuxAttnNorm;
    const void *pb = aux;
    if (t < 64) {
        pb = aux + kAuxONorm + 4 * t;
    } else if (t < 96) {
        const int r = w * kCuQkvg + (t - 64);
        if (r < 3 * kH) pb = aux + kAuxConv + ((size_t)(r / kH) * kH + r % kH) * 4;
    } else if (t < 192) {
        const int j = (t - 96) / 32, r = w * kCuQkvg + (t - 96) % 32;
        if (r < 3 * kH) {
            const uint16_t *tl = reinterpret_cast<const uint16_t *>(p.tails + ((size_t)l * 3 + r / kH) * kTailStripe);
            pb = tl + (size_t)j * kH + ((r % kH) & ~7);
        }
    } else if (t < 196) {
        pb = aux + kAuxALog + 4 * (t - 192);
    } else if (t >= 256 && w < 2 * kNH) {
        pb = p.ab16 + ((size_t)l * 2 * kNH + w) * kH + 8 * (t - 256);
    }
    sd.a = *reinterpret_cast<const f32x4 *>(na + 4 * t);
    sd.m = *reinterpret_cast<const f32x4 *>(aux + kAuxMlpNorm + 4 * t);
    sd.b = *reinterpret_cast<const u32x4 *>(pb);
}

__device__ __forceinline__ void side_commit(const Side &sd, Lds &s, bool lm) {
    const int t = threadIdx.x, w = blockIdx.x;
    *reinterpret_cast<f32x4 *>(s.nw[0] + 4 * t) = sd.a;
    if (lm) return;
    *reinterpret_cast<f32x4 *>(s.nw[1] + 4 * t) = sd.m;
    if (t < 64) {
        *reinterpret_cast<u32x4 *>(s.onw + 4 * t) = sd.b;
    } else if (t < 96) {
        s.taps[t - 64] = __builtin_bit_cast(f32x4, sd.b);
    } else if (t < 192) {
        const int j = (t - 96) / 32, rr = (t - 96) % 32, ch = (w * kCuQkvg + rr) % kH;
        const uint32_t wq[4] = {sd.b.x, sd.b.y, sd.b.z, sd.b.w};
        const uint32_t word = wq[(ch & 7) >> 1];
        s.tails[rr][j] = (ch & 1) ? (word >> 16) : (word & 0xffffu);
    } else if (t < 196) {
        *reinterpret_cast<u32x4 *>(s.scal + 4 * (t - 192)) = sd.b;
    } else if (t >= 256) {
        *reinterpret_cast<u32x4 *>(s.abw + 4 * (t - 256)) = sd.b;
    }
}

// The state tile of (head w / 16, columns 16 (w % 16) ..) of layer l, row t
// (workgroups 0..127, threads 0..255): FP32, or BF16 for REF.  Every thread
// loads (workgroup w >= 128 re-reads the tile of w - 128, thread t >= 256
// row t - 256).
template <int C>
struct Tile {
    static constexpr int NV = C == kRef ? 2 : 4;
    u32x4 v[NV];
};

template <int C>
__device__ __forceinline__ size_t tile_index(int l, int w, int t) {
    return (size_t)l * kNH * kHD * kHD + state_index<true, 16>(w >> 4, t, (w & 15) * 16);
}

template <int C>
__device__ __forceinline__ void tile_issue(Tile<C> &tl, const Params &p, int l) {
    const size_t i = tile_index<C>(l, blockIdx.x & 127, threadIdx.x & 255);
    const u32x4 *src = (C == kRef) ? reinterpret_cast<const u32x4 *>(static_cast<const uint16_t *>(p.state) + i)
                                   : reinterpret_cast<const u32x4 *>(static_cast<const float *>(p.state) + i);
#pragma unroll
    for (int k = 0; k < Tile<C>::NV; ++k) tl.v[k] = src[k];
}

// ---------------------------------------------------------------- stages

// Reads n words of region `src` (tag `tag`) with every wave of the
// workgroup, group (64 words) g by wave g mod 8; f(index, payload) stores
// each word's payload.
template <class F>
__device__ __forceinline__ void xread_all(const uint32_t *src, int n, uint32_t tag, Ctl &c, F f) {
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6), lane = threadIdx.x & 63;
    for (int g = wave; g * 64 < n; g += kNT / 64) {
        const uint32_t pay = xget<64>(src + g * 64, tag, c);
        f(g * 64 + lane, pay);
    }
}


// The same with waves w0, w0 + stride, ... only.
template <class F>
__device__ __forceinline__ void xread_waves(const uint32_t *src, int n, uint32_t tag, Ctl &c, int w0, int stride,
                                            F f) {
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (wave < w0) return;
    for (int g = wave - w0; g * 64 < n; g += stride) {
        const uint32_t pay = xget<64>(src + g * 64, tag, c);
        f(g * 64 + lane, pay);
    }
}

__device__ __forceinline__ void lds_load8(const float *src, float *v) {
    const f32x4 a = reinterpret_cast<const f32x4 *>(src)[0], b = reinterpret_cast<const f32x4 *>(src)[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// Residual add + RMSNorm prologue, the per-kernel step's PRO_RESNORM /
// PRO_EMBED arithmetic: threads 0..255 own elements 8t..8t+7; r = R(res + y)
// (EMBED: the embedding row), res <- r, sixteen-value chunk sums of squares
// added in order, x = R(r * scale * w) into the input lane words.  Returns
// the fast-path verdict.  Every thread calls it (3 barriers).  With fin,
// workgroup 0 also writes the final hidden vector R(x) (the LM head's input).
template <bool EMBED>
__device__ __forceinline__ bool pro_resnorm(Lds &s, const float *w_lds, const u32x4 &e4, const Params &p, WInfo wi,
                                            bool fin) {
    const int t = threadIdx.x;
    const bool act = t < kT;
    float r[8], a[8], b[8];
    PairStats st;
    if (act) {
        if constexpr (EMBED) {
            const uint32_t e[4] = {e4.x, e4.y, e4.z, e4.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                r[2 * j] = u2f(e[j] << 16);
                r[2 * j + 1] = u2f(e[j] & 0xffff0000u);
            }
        } else {
            lds_load8(s.res + 8 * t, a);
            lds_load8(s.y + 8 * t, b);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t rp = cvt_pk(a[2 * j] + b[2 * j], a[2 * j + 1] + b[2 * j + 1]);
                r[2 * j] = u2f(rp << 16);
                r[2 * j + 1] = u2f(rp & 0xffff0000u);
            }
        }
        const float cs = chunk_sumsq8(r);
        if (t & 1) s.scratch[t >> 1] = cs;
    }
    __syncthreads();
    if (t < 64) {
        const f32x4 *s4 = reinterpret_cast<const f32x4 *>(s.scratch);
        float sum = 0.0f;
#pragma unroll 8
        for (int i = 0; i < kH / 64; ++i) {
            const f32x4 c = s4[i];
            sum += c.x;
            sum += c.y;
            sum += c.z;
            sum += c.w;
        }
        if (t == 0) s.bcast[0] = sum;
    }
    __syncthreads();
    const float sum = s.bcast[0];
    if (act) {
        // the stored residual: exact rounding with the canonical NaN when the
        // sum shows a NaN or infinity
        float rs[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) rs[e] = r[e];
        if (!(sum <= 3.402823466e38f)) {
#pragma unroll
            for (int e = 0; e < 8; ++e) rs[e] = EMBED ? rne_bf16(r[e]) : rne_bf16(a[e] + b[e]);
        }
        f32x4 *rd = reinterpret_cast<f32x4 *>(s.res + 8 * t);
        rd[0] = (f32x4){rs[0], rs[1], rs[2], rs[3]};
        rd[1] = (f32x4){rs[4], rs[5], rs[6], rs[7]};
        float w[8];
        lds_load8(w_lds + 8 * t, w);
        const float scale = 1.0f / __builtin_sqrtf(sum / (float)kH + p.eps);
        float xv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) xv[e] = r[e] * scale * w[e];
        uint32_t pairs[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) pairs[j] = cvt_pk(xv[2 * j], xv[2 * j + 1]);
        store_pairs8(s.xs, pairs, st);
        if (fin && blockIdx.x == 0) {
            f32x4 *d = reinterpret_cast<f32x4 *>(p.fhid) + 2 * t;
            float xo[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) xo[e] = rne_bf16(xv[e]);
            d[0] = (f32x4){xo[0], xo[1], xo[2], xo[3]};
            d[1] = (f32x4){xo[4], xo[5], xo[6], xo[7]};
        }
    }
    publish_stats(st, s.red);
    __syncthreads();
    return decide_fast(s.red, wi);
}

// Output norm x gate prologue (PRO_ONORM): per head, the 16 chunk sums of
// squares in order, scale = 1/sqrtf(sum/256 + eps), x = R(a sc w g s(g));
// sigmoid(g) is evaluated here from the exchanged gate, as the QKVG epilogue
// of the per-kernel step evaluates it.  1 barrier.
__device__ __forceinline__ bool pro_onorm(Lds &s, float eps, WInfo wi) {
    const int t = threadIdx.x;
    PairStats st;
    if (t < kT) {
        const int h = t >> 5;
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < kHD / 16; ++i) sum += s.osum[h * (kHD / 16) + i];
        const float sc = 1.0f / __builtin_sqrtf(sum / (float)kHD + eps);
        float a[8], g[8], w[8];
        lds_load8(s.y + 8 * t, a);
        lds_load8(s.g + 8 * t, g);
        lds_load8(s.onw + 8 * (t & 31), w);
        uint32_t pairs[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float sg0 = sigmoid_ref(g[2 * j], Exp2Lds{s.exp2});
            const float sg1 = sigmoid_ref(g[2 * j + 1], Exp2Lds{s.exp2});
            const float x0 = a[2 * j] * sc * w[2 * j] * g[2 * j] * sg0;
            const float x1 = a[2 * j + 1] * sc * w[2 * j + 1] * g[2 * j + 1] * sg1;
            pairs[j] = cvt_pk(x0, x1);
        }
        store_pairs8(s.xs, pairs, st);
    }
    publish_stats(st, s.red);
    __syncthreads();
    return decide_fast(s.red, wi);
}

// The down GEMV's input statistics (PRO_PLAIN): the lane words are already
// in LDS; thread t < 256 scans elements 22t..22t+21 as pairs.  1 barrier.
__device__ __forceinline__ bool pro_plain(Lds &s, WInfo wi) {
    const int t = threadIdx.x;
    constexpr int PER = kI / kT;
    PairStats st;
    if (t < kT) {
#pragma unroll
        for (int j = 0; j < PER / 2; ++j) {
            const uint32_t lo = s.xs[PER * t + 2 * j], hi = s.xs[PER * t + 2 * j + 1];
            st.add((hi & 0xffff0000u) | (lo & 0xffffu));
        }
    }
    publish_stats(st, s.red);
    __syncthreads();
    return decide_fast(s.red, wi);
}

// QKVG epilogue: bank chains of the 32 rows (waves 0..1); conv + SiLU with
// the tail shift for q/k/v rows, the gate for g rows; the q/k rows' partial
// sums of squares (the lower four levels of gdn_tree_reduce_256 per 16-row
// block); workgroups 0..15 finish their a/b row.
template <int C>
__device__ __forceinline__ void epi_qkvg(Lds &s, const Params &p, int l, uint32_t tag) {
    const int t = threadIdx.x, w = blockIdx.x, wave = t >> 6;
    uint32_t *xb = p.xbuf;
    if (t < 128) {
        const float y = chain_rows<kH, kCuQkvg>(s.part);
        float conv_out = 0.0f;
        if ((t & 3) == 0) {
            const int rr = t >> 2, r = w * kCuQkvg + rr;
            const float yv = R<C>(y);
            if (r < 3 * kH) {
                const int kind = r / kH, ch = r - kind * kH;
                const uint32_t b0 = s.tails[rr][0], b1 = s.tails[rr][1], b2 = s.tails[rr][2];
                const float t0 = bf16_bits_to_f32(b0);
                const float t1 = bf16_bits_to_f32(b1);
                const float t2 = bf16_bits_to_f32(b2);
                uint16_t *tl = reinterpret_cast<uint16_t *>(p.tails + ((size_t)l * 3 + kind) * kTailStripe);
                tl[ch] = (uint16_t)b1;
                tl[kH + ch] = (uint16_t)b2;
                tl[2 * kH + ch] = bf16_hi(yv);
                const f32x4 taps = s.taps[rr];
                const float sm = t0 * taps.x + t1 * taps.y + t2 * taps.z + yv * taps.w;
                conv_out = R<C>(silu_ref(sm, Exp2Lds{s.exp2}));
                xput(xb + XQKV + r, tag, bf16_hi(conv_out));
            } else {
                xput(xb + XG + (r - 3 * kH), tag, bf16_hi(yv));
            }
        }
        if (w < 2 * kH / kCuQkvg) {
            const auto add = [](uint32_t x, uint32_t z) { return f2u(u2f(x) + u2f(z)); };
            uint32_t v = f2u(conv_out * conv_out);
            v = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x00, 0xf, 0xf, false);  // quad lane 0
            v = add(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x141, 0xf, 0xf, false));
            v = add(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x140, 0xf, 0xf, false));
            const int lane = t & 63;
            const auto s16 = __builtin_amdgcn_permlane16_swap((int)v, (int)v, false, false);
            v = add(v, (uint32_t)(((lane >> 4) & 1) ? s16[0] : s16[1]));
            const auto s32 = __builtin_amdgcn_permlane32_swap((int)v, (int)v, false, false);
            v = add(v, (uint32_t)((lane >> 5) ? s32[0] : s32[1]));
            if (lane < 2) {  // lane 0: low half, lane 1: high half of the block's sum
                const int idx = 2 * w + wave;
                xput(xb + XQKP + 2 * idx + lane, tag, lane ? (v >> 16) : v);
            }
        }
    }
    if (w < 2 * kNH && t == 3 * 64) {
        float acc = 0.0f;
        for (int j = 0; j < kH / 32; ++j) acc = (acc + s.abpart[2 * j]) + s.abpart[2 * j + 1];
        xput(xb + XAB + w, tag, bf16_hi(R<C>(acc)));
    }
}

// Workgroup w < 16: row w of the tiny a|b projection, FP32 products x * w of
// half-beat t (t < 128), tree16 (gdn_gemv_tiny_ab; the chain runs in the
// epilogue).
__device__ __forceinline__ void ab_products(Lds &s) {
    const int t = threadIdx.x;
    if (blockIdx.x >= 2 * kNH || t >= kHB) return;
    uint32_t xv[16];
    lds_load16u(s.xs + t * 16, xv);
    const u32x4 w0 = *reinterpret_cast<const u32x4 *>(s.abw + 8 * t);
    const u32x4 w1 = *reinterpret_cast<const u32x4 *>(s.abw + 8 * t + 4);
    const uint32_t wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
    float pr[16];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        pr[2 * i] = lane_word_value(xv[2 * i], 0) * u2f(wv[i] << 16);
        pr[2 * i + 1] = lane_word_value(xv[2 * i + 1], 1) * u2f(wv[i] & 0xffff0000u);
    }
    s.abpart[t] = tree16(pr);
}

// Bank chains of 8 rows (wave 0) and the rounded outputs to the exchange.
template <int C, int K>
__device__ __forceinline__ void epi_store8(Lds &s, uint32_t *dst, uint32_t tag) {
    const int t = threadIdx.x;
    if (t < 64) {
        const float y = chain_rows<K, 8>(s.part);
        // lane 4r ends with row r; lanes 32..63 hold no row
        if ((t & 3) == 0 && (t >> 2) < 8) xput(dst + blockIdx.x * 8 + (t >> 2), tag, bf16_hi(R<C>(y)));
    }
}

// gate/up epilogue: chains of the 44 rows (waves 0..2), then SwiGLU over the
// workgroup's 22 channels.  1 barrier.
template <int C>
__device__ __forceinline__ void epi_swiglu(Lds &s, uint32_t *dst, uint32_t tag) {
    const int t = threadIdx.x;
    if (t < 192) {
        const float y = chain_rows<kH, kCuGu>(s.part);
        if ((t & 3) == 0 && (t >> 2) < kCuGu) s.ybuf[t >> 2] = R<C>(y);
    }
    __syncthreads();
    if (t < kCuGu / 2) {
        const float g = s.ybuf[t], u = s.ybuf[t + kCuGu / 2];
        xput(dst + blockIdx.x * (kCuGu / 2) + t, tag, bf16_hi(R<C>(silu_ref(g, Exp2Lds{s.exp2}) * u)));
    }
}

// The gated delta rule for head w / 16, columns 16 (w % 16) .. + 15 (waves
// 0..3 of workgroups 0..127): recur_block's arithmetic (gdn_device.h) with
// its inputs from the exchange, the state tile from registers, and the
// waves joined by an LDS arrival counter instead of the workgroup barrier
// (the other waves read the gate meanwhile).
template <int C>
__device__ __forceinline__ void recur_tile(Lds &s, const Tile<C> &tl, const Params &p, int l, uint32_t tag) {
    constexpr int LDT = kHD + 4;
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int w = blockIdx.x, h = w >> 4, c0 = (w & 15) * 16;
    float *pk_t = s.part, *pq_t = s.part + 16 * LDT;
    Wave4Sync sync{&s.arrive, p.tok + 2};
    float sv[16];
    if constexpr (C == kRef) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t wq[4] = {tl.v[i].x, tl.v[i].y, tl.v[i].z, tl.v[i].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                sv[8 * i + 2 * e] = u2f(wq[e] << 16);
                sv[8 * i + 2 * e + 1] = u2f(wq[e] & 0xffff0000u);
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sv[4 * i] = u2f(tl.v[i].x);
            sv[4 * i + 1] = u2f(tl.v[i].y);
            sv[4 * i + 2] = u2f(tl.v[i].z);
            sv[4 * i + 3] = u2f(tl.v[i].w);
        }
    }
    const float q = s.rq[t], k = s.rk[t];
    const float vi = t < 16 ? s.rv[t] : 0.0f;
    float qv[16], kv[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        qv[i] = s.rqp[i];
        kv[i] = s.rkp[i];
    }
    const float q_sq = tree16(qv), k_sq = tree16(kv);
    const float q_inv = 1.0f / __builtin_sqrtf(q_sq + 1e-6f);
    const float k_inv = 1.0f / __builtin_sqrtf(k_sq + 1e-6f);
    const float qj = q * q_inv, kj = k * k_inv;
    const float qk = wave_tree64(qj * kj);
    if (lane == 0) s.red2[wv] = qk;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        pk_t[e * LDT + t] = sv[e] * kj;
        pq_t[e * LDT + t] = sv[e] * qj;
    }
    sync();
    float acc = 0.0f, pv = 0.0f;
    if (t < 32) {
        const bool is_p = t >= 16;
        const int ci = is_p ? t - 16 : t;
        const f32x4 *src = reinterpret_cast<const f32x4 *>((is_p ? pq_t : pk_t) + ci * LDT);
        // the column in chunks of 16 values, the next chunk read while the
        // current one's adds run
        constexpr int CH = 4;
        f32x4 cur[CH], nxt[CH];
#pragma unroll
        for (int i = 0; i < CH; ++i) cur[i] = src[i];
#pragma unroll
        for (int c4 = 0; c4 < kHD / 4; c4 += CH) {
            if (c4 + CH < kHD / 4) {
#pragma unroll
                for (int i = 0; i < CH; ++i) nxt[i] = src[c4 + CH + i];
            }
#pragma unroll
            for (int i = 0; i < CH; ++i) {
                acc = acc + cur[i].x;
                acc = acc + cur[i].y;
                acc = acc + cur[i].z;
                acc = acc + cur[i].w;
            }
#pragma unroll
            for (int i = 0; i < CH; ++i) cur[i] = nxt[i];
        }
        pv = __int_as_float(
            __builtin_amdgcn_permlane16_swap(__float_as_int(acc), __float_as_int(acc), false, false)[1]);
    } else if (wv == 3) {
        float b_, d_;
        head_scalars(s.rab[0], s.rab[1], s.scal[h], s.scal[kNH + h], b_, d_, Exp2Lds{s.exp2});
        if (lane == 0) {
            s.bd[0] = b_;
            s.bd[1] = d_;
        }
    }
    sync();
    const float beta = s.bd[0], decay = s.bd[1];
    if (t < 32) {
        const bool is_p = t >= 16;
        float o = 0.0f;
        if (!is_p) {
            const float alpha = (s.red2[0] + s.red2[1]) + (s.red2[2] + s.red2[3]);
            const float delta = beta * (vi - decay * acc);
            o = R<C>(0.0625f * (decay * pv + alpha * delta));
            s.dl[t] = delta;
            xput(p.xbuf + XO + h * kHD + c0 + t, tag, bf16_hi(o));
        }
        const uint32_t sq = f2u(o * o);
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) sum += u2f((uint32_t)__builtin_amdgcn_readlane((int)sq, i));
        if (t < 2) xput(p.xbuf + XOSUM + 2 * (h * (kHD / 16) + c0 / 16) + t, tag, t ? (f2u(sum) >> 16) : f2u(sum));
    }
    sync();
    float nv[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) nv[e] = decay * sv[e] + kj * s.dl[e];
    const size_t si = tile_index<C>(l, w, t);
    if constexpr (C == kRef) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            u32x4 v;
            v.x = cvt_pk(nv[8 * i + 0], nv[8 * i + 1]);
            v.y = cvt_pk(nv[8 * i + 2], nv[8 * i + 3]);
            v.z = cvt_pk(nv[8 * i + 4], nv[8 * i + 5]);
            v.w = cvt_pk(nv[8 * i + 6], nv[8 * i + 7]);
            bool special = false;
#pragma unroll
            for (int e = 0; e < 8; ++e) special |= !(fabsf(nv[8 * i + e]) <= 3.402823466e38f);
            if (special) {  // a NaN or infinity: the integer rounding (canonical NaN)
                uint32_t pk[4];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    pk[e] = (f2u(rne_bf16(nv[8 * i + 2 * e])) >> 16) |
                            (f2u(rne_bf16(nv[8 * i + 2 * e + 1])) & 0xffff0000u);
                v.x = pk[0]; v.y = pk[1]; v.z = pk[2]; v.w = pk[3];
            }
            reinterpret_cast<u32x4 *>(static_cast<uint16_t *>(p.state) + si)[i] = v;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f32x4 v;
            v.x = nv[4 * i + 0]; v.y = nv[4 * i + 1]; v.z = nv[4 * i + 2]; v.w = nv[4 * i + 3];
            reinterpret_cast<f32x4 *>(static_cast<float *>(p.state) + si)[i] = v;
        }
    }
}

// The recurrence's inputs for head w / 16, columns 16 (w % 16) ..: q and k
// of the head (waves 0..3 and 4..7); then waves 0..3 read the 16 columns of
// v, the head's q and the k partial sums of squares, and a and b.
__device__ __forceinline__ void recur_inputs(Lds &s, const Params &p, uint32_t tag, Ctl &c) {
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int w = blockIdx.x, h = w >> 4, c0 = (w & 15) * 16;
    const uint32_t *xb = p.xbuf;
    if (wave >= 4) {
        const uint32_t pay = xget<64>(xb + XQKV + kH + h * kHD + 64 * (wave - 4), tag, c);
        s.rk[64 * (wave - 4) + lane] = u2f(pay << 16);
        return;
    }
    {
        const uint32_t pay = xget<64>(xb + XQKV + h * kHD + 64 * wave, tag, c);
        s.rq[64 * wave + lane] = u2f(pay << 16);
    }
    if (wave == 0) {
        const uint32_t pay = xget<16>(xb + XQKV + 2 * kH + h * kHD + c0, tag, c);
        if (lane < 16) s.rv[lane] = u2f(pay << 16);
    } else if (wave == 1 || wave == 2) {
        const uint32_t *base = xb + XQKP + (wave == 2 ? 256 : 0) + 32 * h;
        float *dst = wave == 2 ? s.rkp : s.rqp;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const uint32_t pay = xget<16>(base + 16 * half, tag, c);
            const float v = join_halves(pay);
            if (lane < 16 && (lane & 1) == 0) dst[8 * half + (lane >> 1)] = v;
        }
    } else {
        const uint32_t pay = xget<16>(xb + XAB, tag, c);
        if (lane == h) s.rab[0] = u2f(pay << 16);
        if (lane == kNH + h) s.rab[1] = u2f(pay << 16);
    }
}

// LM-head epilogue: chains of the 125 rows (waves 0..7), FP32 logits, the
// workgroup's argmax in row order (strict '>' per lane, merges keep the
// larger value and on ties the lower index).  1 barrier.
__device__ __forceinline__ void epi_lm(Lds &s, const Params &p, uint32_t tag) {
    const int t = threadIdx.x, w = blockIdx.x;
    const int row0 = w * kLmRows;
    if (t < 512) {
        const float y = chain_rows<kH, kLmRows>(s.part);
        if ((t & 3) == 0 && (t >> 2) < kLmRows) {
            p.logits[row0 + (t >> 2)] = y;
            s.ybuf[t >> 2] = y;
        }
    }
    __syncthreads();
    if (t < 64) {
        float best = -3.402823466e38f;
        int idx = 0;
        for (int i = t; i < kLmRows; i += 64) {
            const float v = s.ybuf[i];
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
        if (t < 4) {
            const uint32_t word = t < 2 ? f2u(best) : (uint32_t)idx;
            xput(p.xbuf + XARG + 4 * w + t, tag, (t & 1) ? (word >> 16) : word);
        }
    }
}

// Workgroup 0: the 256 workgroup results in index order (k_argmax's
// merge), then the token to mapped host memory.  2 barriers.
__device__ __forceinline__ void argmax_merge(Lds &s, const Params &p, uint32_t tag, Ctl &c) {
    const int t = threadIdx.x;
    xread_all(p.xbuf + XARG, 4 * kWG, tag, c, [&](int i, uint32_t pay) { s.xs[i] = pay; });
    __syncthreads();
    if (t < kT) {
        s.av[t] = u2f(s.xs[4 * t] | (s.xs[4 * t + 1] << 16));
        s.ai[t] = (int)(s.xs[4 * t + 2] | (s.xs[4 * t + 3] << 16));
    }
    __syncthreads();
    if (t < kT) {
        float best = -3.402823466e38f;
        int idx = 0;
        const float v = s.av[t];
        if (v > best) {
            best = v;
            idx = s.ai[t];
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
        const int lane = t & 63, wv = t >> 6;
        if (lane == 0) {
            s.bcast[wv] = best;
            s.red[wv] = (uint32_t)idx;
        }
    }
    __syncthreads();
    if (t == 0) {
        float best = s.bcast[0];
        int idx = (int)s.red[0];
        for (int i = 1; i < 4; ++i) {
            const float bv = s.bcast[i];
            const int bi = (int)s.red[i];
            if (bv > best || (bv == best && bi < idx)) {
                best = bv;
                idx = bi;
            }
        }
        // a wait that ran out anywhere in the grid (its abort word is in
        // memory before that workgroup's last exchange words) fails the step
        if (sload1(c.abort_word) == c.abort_val) __hip_atomic_store(p.tok + 2, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __hip_atomic_store(p.tok + 1, idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

// ------------------------------------------------------------ the kernel

// Phase stamp k of layer l (the LM head is layer `layers`) from thread 0.
__device__ __forceinline__ void stamp(const Params &p, int l, int k) {
    if (p.stamps != nullptr && threadIdx.x == 0)
        p.stamps[((size_t)blockIdx.x * (kMaxLayers + 1) + l) * kStamps + k] = __builtin_amdgcn_s_memrealtime();
}

template <int C>
__global__ __launch_bounds__(kNT, 1) void k_step(const Params p) {
    static_assert(C == kRef || C == kBf16w, "BF16 contracts");
    __shared__ Lds s;
    const int t = threadIdx.x, w = blockIdx.x;
    uint32_t *xb = p.xbuf;
    Ctl c{xb + XABORT, p.tok + 2, 0xAB000000u | (p.tag0 & 0xffffu), false};
    const char *lm = static_cast<const char *>(p.w_lm) + (size_t)w * items_of(SL) * 32;

    // the token and its embedding row, layer 0's small weights
    int tok = p.tok[0];
    if (tok < 0 || tok >= kWG * kLmRows) tok = 0;  // the host rejects these first
    const u32x4 e4 =
        *reinterpret_cast<const u32x4 *>(static_cast<const uint16_t *>(p.w_emb) + (size_t)tok * kH + 8 * (t & (kT - 1)));
    Side sd;
    side_issue(sd, p, 0, false);
    fill_exp2_lds_imm(s.exp2);
    side_commit(sd, s, false);
    __syncthreads();

    Ring ring;
    bool fast;
    for (int l = 0; l < p.layers; ++l) {
        const bool last = l + 1 == p.layers;
        const Slices cur = slices_of(p, l);
        // this layer's state tile, then its first kD weight items: both in
        // flight while the layer's input arrives
        Tile<C> tl;
        stamp(p, l, 0);
        tile_issue<C>(tl, p, l);
        prime<SQ, 0>(ring, slice_sel<SQ>(cur));

        // ---- QKVG
        if (l == 0) {
            fast = pro_resnorm<true>(s, s.nw[0], e4, p, p.i_qkvg[0], false);
        } else {
            xread_all(xb + XYD, kH, tag_of(p.tag0, l - 1, XK_DOWN), c,
                      [&](int i, uint32_t pay) { s.y[i] = u2f(pay << 16); });
            __syncthreads();
            fast = pro_resnorm<false>(s, s.nw[0], u32x4{}, p, p.i_qkvg[l], false);
        }
        stamp(p, l, 1);
        ab_products(s);
        proc_stage<0, 7>(fast, ring, cur, s.xs, s.part);
        __syncthreads();
        stamp(p, l, 2);
        const uint32_t tq = tag_of(p.tag0, l, XK_QKVG);
        epi_qkvg<C>(s, p, l, tq);
        stamp(p, l, 3);

        // ---- recurrence (workgroups 0..127), the gate everywhere
        if (w < 128) recur_inputs(s, p, tq, c);
        if (t == 0) s.arrive = 0;
        __syncthreads();
        stamp(p, l, 4);
        const uint32_t tr = tag_of(p.tag0, l, XK_RECUR);
        if (w < 128 && t < kT) recur_tile<C>(s, tl, p, l, tr);
        stamp(p, l, 5);
        xread_waves(xb + XG, kH, tq, c, 4, 4, [&](int i, uint32_t pay) { s.g[i] = u2f(pay << 16); });

        // ---- o_proj
        xread_all(xb + XO, kH + 256, tr, c, [&](int i, uint32_t pay) {
            const float v = join_halves(pay);
            if (i < kH) s.y[i] = u2f(pay << 16);
            else if (((i - kH) & 1) == 0) s.osum[(i - kH) >> 1] = v;
        });
        __syncthreads();
        stamp(p, l, 6);
        fast = pro_onorm(s, p.eps, p.i_o[l]);
        proc_stage<8, 9>(fast, ring, cur, s.xs, s.part);
        __syncthreads();
        stamp(p, l, 7);
        const uint32_t to = tag_of(p.tag0, l, XK_OPROJ);
        epi_store8<C, kH>(s, xb + XYO, to);

        // ---- gate/up
        xread_all(xb + XYO, kH, to, c, [&](int i, uint32_t pay) { s.y[i] = u2f(pay << 16); });
        __syncthreads();
        fast = pro_resnorm<false>(s, s.nw[1], u32x4{}, p, p.i_gu[l], false);
        stamp(p, l, 8);
        proc_stage<10, 20>(fast, ring, cur, s.xs, s.part);
        __syncthreads();
        stamp(p, l, 9);
        const uint32_t tg = tag_of(p.tag0, l, XK_SWIGLU);
        epi_swiglu<C>(s, xb + XH, tg);

        // ---- down; the next layer's (or the LM head's) small weights are
        // issued here and committed once the products are done
        side_issue(sd, p, last ? l : l + 1, last);
        xread_all(xb + XH, kI, tg, c, [&](int i, uint32_t pay) { s.xs[i] = (i & 1) ? (pay << 16) : pay; });
        __syncthreads();
        fast = pro_plain(s, p.i_down[l]);
        stamp(p, l, 10);
        proc_stage<21, 27>(fast, ring, cur, s.xs, s.part);
        side_commit(sd, s, last);
        __syncthreads();
        stamp(p, l, 11);
        epi_store8<C, kI>(s, xb + XYD, tag_of(p.tag0, l, XK_DOWN));
        stamp(p, l, 12);
    }

    // ---- final norm, LM head, argmax
    stamp(p, p.layers, 0);
    prime<SL, 0>(ring, lm);
    xread_all(xb + XYD, kH, tag_of(p.tag0, p.layers - 1, XK_DOWN), c,
              [&](int i, uint32_t pay) { s.y[i] = u2f(pay << 16); });
    __syncthreads();
    fast = pro_resnorm<false>(s, s.nw[0], u32x4{}, p, p.i_lm, true);
    stamp(p, p.layers, 1);
    {
        uint32_t xv[16];
        lds_load16u(s.xs + (t % kHB) * 16, xv);
        proc_lm_range<0, kSlotsLm - 1>(ring, lm, s.xs, s.part, xv, fast);
    }
    __syncthreads();
    stamp(p, p.layers, 2);
    const uint32_t ta = tag_of(p.tag0, p.layers, XK_ARGMAX);
    epi_lm(s, p, ta);
    stamp(p, p.layers, 3);
    if (w == 0) argmax_merge(s, p, ta, c);
    stamp(p, p.layers, 4);
}

}  // namespace pst

// ------------------------------------------------------------ host side

int persist_launch(int contract, const pst::Params &p, hipStream_t s) {
    void *args[] = {const_cast<pst::Params *>(&p)};
    const void *fn = contract == kRef ? reinterpret_cast<const void *>(&pst::k_step<kRef>)
                                      : reinterpret_cast<const void *>(&pst::k_step<kBf16w>);
    GDN_HIP(hipLaunchCooperativeKernel(fn, dim3(pst::kWG), dim3(pst::kNT), args, 0, s));
    return 0;
}

bool persist_supported(int contract) {
    if (contract != kRef && contract != kBf16w) return false;
    int dev = 0, coop = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess) return false;
    if (hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess || !coop) return false;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return false;
    const void *fn = contract == kRef ? reinterpret_cast<const void *>(&pst::k_step<kRef>)
                                      : reinterpret_cast<const void *>(&pst::k_step<kBf16w>);
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, pst::kNT, 0) != hipSuccess) return false;
    return (long)per_cu * cus >= pst::kWG;
}

namespace {
std::mutex g_xbuf_mu;
std::vector<std::pair<int, uint32_t *>> g_xbuf_pool;  // released areas: (device, address)
std::vector<std::pair<uint32_t *, int>> g_xbuf_dev;   // every area's device
}  // namespace

uint32_t *persist_xbuf_acquire() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return nullptr;
    uint32_t *x = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_xbuf_mu);
        for (size_t i = 0; i < g_xbuf_pool.size(); ++i) {
            if (g_xbuf_pool[i].first == dev) {
                x = g_xbuf_pool[i].second;
                g_xbuf_pool.erase(g_xbuf_pool.begin() + (long)i);
                break;
            }
        }
    }
    if (x == nullptr) {
        if (hipExtMallocWithFlags(reinterpret_cast<void **>(&x), (size_t)pst::XWORDS * 4, hipDeviceMallocUncached) !=
            hipSuccess)
            return nullptr;
        std::lock_guard<std::mutex> lk(g_xbuf_mu);
        g_xbuf_dev.push_back({x, dev});
    }
    // every word's tag 0xffff, which no step uses; complete before the
    // run state's first launch (its stream does not wait for this one)
    if (hipMemset(x, 0xff, (size_t)pst::XWORDS * 4) != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
        persist_xbuf_release(x);
        return nullptr;
    }
    return x;
}

void persist_xbuf_release(uint32_t *xbuf) {
    if (xbuf == nullptr) return;
    std::lock_guard<std::mutex> lk(g_xbuf_mu);
    for (const auto &d : g_xbuf_dev)
        if (d.first == xbuf) {
            g_xbuf_pool.push_back({d.second, xbuf});
            return;
        }
}

}  // namespace gdn

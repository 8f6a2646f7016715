// gdn_persist.h -- the persistent decode step of the batch-1 engine: one
// cooperative launch of 256 one-per-CU workgroups runs a whole token (every
// layer, the LM head and the argmax).  Shared by gdn_engine.hip (which owns
// the run state and launches it) and gdn_persist.hip (the kernel).  Not part
// of the ABI.
#ifndef GDN_PERSIST_H
#define GDN_PERSIST_H

#include <hip/hip_runtime.h>

#include <cstdint>

#include "gdn_gemv.h"

namespace gdn {
namespace pst {

constexpr int kWG = 256;    // workgroups: one per CU
constexpr int kNT = 512;    // threads per workgroup (8 waves, 256 VGPRs each), every one a weight-stream thread
constexpr int kLmRows = 125;  // LM-head rows per workgroup: the step runs vocabularies of 256 x 125

// Exchange area (32-bit words in uncached device memory).  Every value a
// stage hands to another workgroup is one word (tag << 16) | 16-bit payload:
// a BF16 value, or one half of an FP32 value (low half first).  A reader
// accepts a word when its tag is the exchange's tag for this step, so no
// flag, fence or reset is needed; the 16-bit payload halves keep every word
// self-describing.  Offsets are multiples of 64 words (4 scalar lines).
constexpr int XQKV = 0;                 // q, k, v after conv + SiLU [3][2048]
constexpr int XG = XQKV + 3 * kH;       // gate g [2048]
constexpr int XQKP = XG + kH;           // q/k partial sums of squares [2][8][16], FP32
constexpr int XAB = XQKP + 2 * 256;     // a[8], b[8] (BF16-valued)
constexpr int XO = XAB + 64;            // recurrence output o [2048]
constexpr int XOSUM = XO + kH;          // output-norm chunk sums [8][16], FP32
constexpr int XYO = XOSUM + 2 * 128;    // o_proj output [2048]
constexpr int XH = XYO + kH;            // SwiGLU output [5632]
constexpr int XYD = XH + kI;            // down output [2048]
constexpr int XARG = XYD + kH;          // per-workgroup argmax [256][value lo, hi, index lo, hi]
constexpr int XABORT = XARG + 4 * kWG;  // [0]: the abort word of a step whose wait ran out
constexpr int XWORDS = XABORT + 64;

// Exchange kinds; the tag of kind x in layer l (the LM head is layer L) is
// (tag0 + 8 l + x) mod 2^16, tag0 a multiple of 256 that advances by 256 per
// step, so no tag repeats in a buffer word between two writes and none is
// 0xffff (the words start as 0xffffffff).
enum { XK_QKVG = 0, XK_RECUR = 1, XK_OPROJ = 2, XK_SWIGLU = 3, XK_DOWN = 4, XK_ARGMAX = 5 };

struct Params {
    const void *w_qkvg[kMaxLayers], *w_o[kMaxLayers], *w_gu[kMaxLayers], *w_down[kMaxLayers];
    WInfo i_qkvg[kMaxLayers], i_o[kMaxLayers], i_gu[kMaxLayers], i_down[kMaxLayers];
    const void *w_lm;
    WInfo i_lm;
    const void *w_emb;
    const float *aux;       // [layers][kAuxLayer] + final norm
    const uint16_t *ab16;   // [layers][16][kH]
    void *state;            // [layers][8] tiles (FP32, or BF16 for REF)
    float *tails;           // [layers][3] stripes
    uint32_t *xbuf;         // exchange area (uncached)
    float *logits, *fhid, *resid, *xrow;
    int *tok;               // device address of the mapped words: [0] in, [1] out, [2] error
    int layers;
    float eps;
    uint32_t tag0;
    // phase stamps (100 MHz real-time counter) of every workgroup's thread 0,
    // [kWG][kMaxLayers + 1][kStamps], or null
    uint64_t *stamps;
};
constexpr int kStamps = 16;

}  // namespace pst

// Launches one persistent step on stream s (cooperative: all 256 workgroups
// co-resident).  contract is GDN_CONTRACT_REF or GDN_CONTRACT_BF16W_FP32S.
int persist_launch(int contract, const pst::Params &p, hipStream_t s);
// Whether this device can hold the persistent step's grid at once.
bool persist_supported(int contract);
// An exchange area on the calling device for one run state: uncached
// memory, initialised to 0xffffffff.  Areas are never freed (uncached
// memory that a kernel has read is kept until the process ends): release
// returns one to a per-device pool that acquire reuses.  nullptr if the
// allocation fails.
uint32_t *persist_xbuf_acquire();
void persist_xbuf_release(uint32_t *xbuf);

}  // namespace gdn

#endif

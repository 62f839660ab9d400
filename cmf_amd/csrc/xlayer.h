// XCD-partitioned decoder blocks (xlayer.hip): one Qwen3-arch block of the
// verify / draft forward as two launches of 8 x 32 workgroups, the
// workgroups of XCD x (blockIdx % 8) cooperating through that XCD's L2.
#pragma once

#include "common.h"

namespace cmf {

constexpr int XL_XCD = 8;     // XCDs of an MI355X (workgroup i runs on XCD i % 8)
constexpr int XL_WG = 32;     // workgroups per XCD (one per CU)
constexpr int XL_T = 512;     // threads per workgroup
constexpr int XL_BT = 6;      // attention: 16-position tiles held per workgroup
constexpr int XL_NQ = 32;     // attention: queries (rows x query heads per kv head)
constexpr int XL_E2S = 132;   // attention partial: m, l, o[128] (+ pad), tagged pairs

// Device buffers shared by every block of a model (allocated once).
struct XlBufs {
    uint64_t *e0 = nullptr, *e1 = nullptr, *e2 = nullptr, *e3 = nullptr;  // tagged exchange areas
    float *pa = nullptr, *pb = nullptr;  // per-XCD residual partials [8][MAXB][H] (attention, FFN)
    float *ha = nullptr, *hb = nullptr;  // residual rows [MAXB][H] (ping-pong)
    uint32_t* gen = nullptr;             // sequence generation (tags), bumped by xl_finish
    // nonzero: bit 1 an exchange wait gave up, bit 4 more attention positions
    // than the launch's bound, bit 8 two workgroups of a launch claimed one
    // (XCD, index) slot (a workgroup ran off its XCD)
    int* err = nullptr;
    uint32_t* claim = nullptr;           // [8][32] launch tag per (XCD, index) slot
    int e0s = 0, e1s = 0;                // row strides (pairs) of e0 / e1
};

struct XlShape {
    int H, I, nh, nkv, hd, max_seq;
    double eps;
};

struct XlAttnW {
    const void *wqkv, *sqkv;  // q8 [(nh + 2 nkv) hd][H]
    const void *wo, *so;      // q8 [H][nh hd]
    int nkc_qkv, nkc_o;
    const float *in_norm, *qn, *kn;
    float *kc, *vc;
};
struct XlFfnW {
    const void *wgu, *sgu;    // q4t, gate/up rows interleaved 8 / 8 per row block [2 I][H]
    const void *wdn, *sdn;    // q4t [H][I]
    int ntg_gu, ntg_dn;
    const float* post_norm;
};

// An MI355X as these launches assume it: gfx950 with 8 XCDs x 32 CUs, a
// launch's workgroups dispatched round-robin over the XCDs.
bool xl_device_fits();
// Whether the shape (and the device) can take the XCD-partitioned blocks for
// batches of up to nb rows and attention over up to max_len positions.
bool xl_shape_ok(const XlShape& s, int nb, int max_len);
size_t xl_bytes(const XlShape& s);
int xl_alloc(XlBufs& b, const XlShape& s, void* (*alloc)(void*, size_t), void* ctx);

// Block li of a sequence (li counts the blocks of one forward: 0, 1, ...).
// Block 0 reads the residual rows h0; block li > 0 reads hb plus the
// previous block's FFN partials.  The attention launch writes its input
// rows to ha and leaves its output projection as partials pa; the FFN launch
// writes h_mid = ha + sum(pa) to hb and leaves the down projection as
// partials pb, until the next block or xl_finish adds them.
// max_len bounds the positions after the block's rows (as xl_shape_ok).
int xl_block(const XlBufs& b, const XlShape& s, const XlAttnW& aw, const XlFfnW& fw, const float* h0, int nb,
             const int* pbase, int padd, int max_len, const float2* rope, int li, hipStream_t st);
// hout = hb + sum(pb) (the sequence's output rows); next generation.
void xl_finish(const XlBufs& b, const XlShape& s, float* hout, int nb, hipStream_t st);
// Exchange areas and claim slots zeroed, generation 1 (stream-ordered): run
// before the 32-bit tags (generation * 256 + call) could repeat.
void xl_reset(const XlBufs& b, hipStream_t st);
constexpr uint32_t XL_GEN_RESET = 1u << 22;  // generations after which the host resets

}  // namespace cmf

// Runtime internals shared by runtime.hip and engine.hip.
#pragma once

#include <vector>

#include "../../include/cmf_hip.h"
#include "common.h"

namespace cmf {

hipStream_t stream();
int device();
int ensure_init();

// Sources of a q4t / q4tp tensor, one entry per device row (concatenation of
// several tensors along rows is expressed by appending their rows).
struct Q4Src {
    int dtype = 0;
    int rows = 0, cols = 0;
    std::vector<const uint8_t*> rowbase;  // q4t: 18-byte tiles; q4tp: 16-byte nibble tiles
    std::vector<const uint8_t*> codes;    // q4tp: the row's 5-bit code bytes
    std::vector<const uint8_t*> params;   // q4tp: the row's (f16 lo, f16 step)
    size_t code_stride = 0;
};

int build_q8(DevWeight& w, int rows, int cols, const int8_t* const* rowptr, const float* rs);
int build_q4(DevWeight& w, const Q4Src& src);
int fill_q4src(Q4Src& s, int dtype, int rows, int cols, const uint8_t* payload, int row_offset);
// gate and up [I x cols] (same dtype) as one weight of 2I rows whose row
// blocks hold 8 gate rows then the 8 matching up rows (I % 8 == 0)
int build_swiglu(DevWeight& w, const cmf_tensor* g, const cmf_tensor* u);
void free_weight(DevWeight& w);

}  // namespace cmf

struct cmf_moe_s;
namespace cmf {
struct XSrc;
// The MoE layer (moe.hip) as the decode engine drives it: descriptors
// uploaded (before any capture), then routing + experts of b <= 16 rows of
// the operand producer x on the stream, out [b][ldo] (resid: +=).
int moe_prepare(cmf_moe_s* m);
int moe_hidden(cmf_moe_s* m);
int moe_experts_count(cmf_moe_s* m);
int moe_ffn_launch(cmf_moe_s* m, const XSrc& x, const float* d_logits, int b, float* d_out, int ldo, bool resid,
                   hipStream_t s);

}  // namespace cmf
